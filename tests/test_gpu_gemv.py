"""GPU parity of the quantised products, through the C-ABI.

Bars: Q8 activation blocks and block dequantisation bit-exact with the
oracle; matvec / matbatch / lm_head within 1e-3 relative L2 of the oracle's
fp32 results on the same seeded inputs.  matvec keeps the integer block dots
(only fp32 accumulation order differs: ~1e-7).  matbatch of quantised weights
runs on fp16 matrix cores with both operands as fp16 (hi, lo) pairs, three
products per K slice, which is held to 1e-5 (measured ~2e-7): a kernel that
dropped a lo term, or rounded either operand to one fp16, lands near 3e-4."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import synth
from conftest import gncx, ptr, rel_l2

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 2, 8, 12, 14, 30
TOL = 1e-3  # relative L2, fp32 outputs
TOL_MATBATCH = 1e-5  # the fp16-pair products of matbatch (quantised types)


def test_act_quant_bitexact(lib, oracle):
    rows, k = 3, 4096
    x = synth.make_activations(rows, k, seed=1).copy()
    x[0, 64:96] = 0.0
    x[1, 0] = 127.0
    x[1, 1:5] = [2.5, 3.5, -2.5, -0.5]
    x[2, 100:132] *= 1e-30  # tiny values
    q = np.zeros(rows * k, np.int8)
    meta = np.zeros((rows * k // 32, 4), np.int32)
    lib.gncx_hip_quantize_act(ptr(x), rows, k, ptr(q), ptr(meta))
    gncx.check(lib)
    want = np.concatenate([oracle.quantize_act(x[r]) for r in range(rows)])
    assert np.array_equal(q.reshape(-1, 32), want["qs"])
    assert np.array_equal(meta[:, 0].view(np.float32), want["d"])
    assert np.array_equal(meta[:, 1], want["sum_lo16"])
    assert np.array_equal(meta[:, 2], want["sum_hi16"])
    assert np.array_equal(meta[:, 3], want["sum"])


@pytest.mark.parametrize("t,k,n", [(Q4_0, 4096, 64), (Q8_0, 4096, 64), (Q4_K, 4096, 64), (Q6_K, 4096, 64),
                                   (Q6_K, 14336, 16), (BF16, 1024, 32)])
def test_dequant_bitexact(lib, oracle, t, k, n):
    w = synth.make_weights(t, n, k, seed=10 + t)
    out = np.zeros((n, k), np.float32)
    lib.gncx_hip_dequantize(ptr(w), 0, t, k, n, ptr(out))
    gncx.check(lib)
    assert np.array_equal(out, oracle.dequant(t, w, k, n, gncx.row_bytes(t, k)))


def test_fp16_scales_all_codes(lib, oracle):
    """Every fp16 code as a Q8_0 block scale with q = 1: the device decode of
    the scale must equal the IEEE value (subnormals included)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(codes.view(np.float16))
    codes = codes[finite]
    n = codes.size
    blocks = np.zeros((n, 34), np.uint8)
    blocks[:, 0:2] = codes.view(np.uint8).reshape(n, 2)
    blocks[:, 2] = 1
    out = np.zeros((n, 32), np.float32)
    lib.gncx_hip_dequantize(ptr(blocks.reshape(-1)), 0, Q8_0, 32, n, ptr(out))
    gncx.check(lib)
    assert np.array_equal(out[:, 0], codes.view(np.float16).astype(np.float32))


# config shapes: Q4_0 4096->4096, Llama/Qwen decode GEMVs, small BF16
MATVEC_CASES = [
    (Q4_0, 4096, 4096), (Q4_K, 4096, 14336), (Q6_K, 14336, 4096), (Q8_0, 4096, 4096), (Q4_K, 4096, 4096),
    (Q4_K, 12288, 4096), (Q6_K, 4096, 2048), (Q4_0, 1024, 333), (Q8_0, 96, 7), (Q4_K, 256, 1),
    (Q6_K, 512, 65), (BF16, 4096, 512),
    # rows split into 3 to 7 K-slices under each schedule, ragged row counts
    (Q8_0, 14336, 4099), (Q4_K, 14336, 1000), (Q6_K, 12288, 777), (Q4_K, 12288, 12288),
]


@pytest.mark.parametrize("t,k,n", MATVEC_CASES)
def test_matvec_parity(lib, oracle, t, k, n):
    w = synth.make_weights(t, n, k, seed=1000 + t + k + n)
    x = synth.make_activations(1, k, seed=2000 + t + k + n)
    y = np.full(n, np.nan, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, t, ptr(x), None, k, n, ptr(y), None)
    gncx.check(lib)
    err = rel_l2(y, oracle.matvec(t, w, x, k, n))
    print(f"matvec type={t} k={k} n={n} rel_l2={err:.3e}")
    assert err < TOL


def test_matvec_lm_head_shape(lib, oracle):
    """Q6_K 4096 -> 128256 (the Llama-3 lm_head GEMV)."""
    t, k, n = Q6_K, 4096, 128256
    w = synth.make_weights(t, n, k, seed=77)
    x = synth.make_activations(1, k, seed=78)
    y = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, t, ptr(x), None, k, n, ptr(y), None)
    gncx.check(lib)
    err = rel_l2(y, oracle.matvec(t, w, x, k, n))
    print(f"lm_head-shaped matvec rel_l2={err:.3e}")
    assert err < TOL
    lib.gncx_hip_weight_forget(ptr(w))


@pytest.mark.parametrize("name,t", [("q4_0", Q4_0), ("q8_0", Q8_0), ("q4_k", Q4_K), ("q6_k", Q6_K), ("bf16", BF16)])
def test_matvec_matbatch_vs_reference_vectors(lib, golden, name, t):
    k, n, b = int(golden["mv_k"]), int(golden["mv_n"]), int(golden["mv_b"])
    # arrays whose address is passed must stay referenced until the call returns
    w = golden[f"{name}_w"].copy()
    x = golden[f"{name}_x"].copy()
    xb = golden[f"{name}_xb"].copy()
    y = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, t, ptr(x), None, k, n, ptr(y), None)
    gncx.check(lib)
    assert rel_l2(y, golden[f"{name}_y"]) < TOL
    yb = np.zeros((b, n), np.float32)
    lib.gncx_xfold_universal_matbatch(ptr(w), 0, t, ptr(xb), b, k, n, ptr(yb), None)
    gncx.check(lib)
    assert rel_l2(yb, golden[f"{name}_yb"]) < TOL


def test_matvec_edge_cases(lib, oracle):
    k, n = 512, 40
    w = synth.make_weights(Q4_K, n, k, seed=5)
    # all-zero activations: every block has d = 0 -> exact zeros
    y = np.full(n, 3.0, np.float32)
    z = np.zeros(k, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, ptr(z), None, k, n, ptr(y), None)
    gncx.check(lib)
    assert not y.any()
    # unknown ggml type: output untouched (cpp:1362-1462), no error
    y[:] = 5.0
    lib.gncx_xfold_universal_matvec(ptr(w), 0, 99, ptr(z), None, k, n, ptr(y), None)
    assert np.all(y == 5.0)
    assert lib.gncx_hip_last_status() == 0
    # weights addressed by (base, offset) inside a larger buffer
    pad = np.zeros(4096 + w.size, np.uint8)
    pad[4096:] = w
    x = synth.make_activations(1, k, seed=6)
    y2 = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(pad), 4096, Q4_K, ptr(x), None, k, n, ptr(y2), None)
    gncx.check(lib)
    assert rel_l2(y2, oracle.matvec(Q4_K, w, x, k, n)) < TOL


def test_weight_cache_detects_rewritten_host_buffer(lib, oracle):
    k, n = 1024, 64
    w = synth.make_weights(Q6_K, n, k, seed=7)
    x = synth.make_activations(1, k, seed=8)
    y = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q6_K, ptr(x), None, k, n, ptr(y), None)
    w[:] = synth.make_weights(Q6_K, n, k, seed=9)  # same address, new content
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q6_K, ptr(x), None, k, n, ptr(y), None)
    gncx.check(lib)
    assert rel_l2(y, oracle.matvec(Q6_K, w, x, k, n)) < TOL


def test_weight_cache_reads_only_the_calls_range(lib, oracle):
    """A weight copy is keyed by host address; when the memory there is now a
    smaller allocation (a freed array whose address came back), the cache
    check must read only the bytes this call names.  Here the tail of the
    first call's mapping is unmapped before a call with fewer rows at the same
    address: a check over the first call's size would read unmapped pages."""
    libc = C.CDLL(None, use_errno=True)
    libc.mmap.restype = C.c_void_p
    libc.mmap.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_long]
    libc.munmap.argtypes = [C.c_void_p, C.c_size_t]
    k, n_big, n_small = 256, 1024, 256  # 144-byte rows: 36 and 9 pages of 4 KiB
    rb = 144
    big, small = n_big * rb, n_small * rb
    assert small % 4096 == 0
    addr = libc.mmap(None, big, 0x1 | 0x2, 0x02 | 0x20, -1, 0)  # PROT_READ|WRITE, MAP_PRIVATE|ANONYMOUS
    assert addr not in (None, C.c_void_p(-1).value)
    mapped = big
    try:
        w = synth.make_weights(Q4_K, n_big, k, seed=71)
        C.memmove(addr, w.ctypes.data, big)
        x = synth.make_activations(1, k, seed=72)
        y = np.zeros(n_big, np.float32)
        lib.gncx_xfold_universal_matvec(C.c_void_p(addr), 0, Q4_K, ptr(x), None, k, n_big, ptr(y), None)
        gncx.check(lib)
        assert rel_l2(y, oracle.matvec(Q4_K, w, x, k, n_big)) < TOL
        assert libc.munmap(C.c_void_p(addr + small), big - small) == 0
        mapped = small
        ys = np.zeros(n_small, np.float32)
        lib.gncx_xfold_universal_matvec(C.c_void_p(addr), 0, Q4_K, ptr(x), None, k, n_small, ptr(ys), None)
        gncx.check(lib)
        assert rel_l2(ys, oracle.matvec(Q4_K, w[:small], x, k, n_small)) < TOL
    finally:
        lib.gncx_hip_weight_forget(C.c_void_p(addr))
        libc.munmap(C.c_void_p(addr), mapped)


def test_activation_cache_follows_reference_rule(lib, oracle):
    """With in_tokens given, the same in_vec pointer and no new norm epoch,
    the reference reuses its quantised activations (cpp:1345) -- even when
    the host vector changed in between; the library keeps that behaviour."""
    k, n = 512, 32
    w = synth.make_weights(Q4_K, n, k, seed=10)
    x = synth.make_activations(1, k, seed=11)
    x0 = x.copy()
    toks = (gncx.GNCXCompactToken * k)()
    y1 = np.zeros(n, np.float32)
    y2 = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, ptr(x), C.addressof(toks), k, n, ptr(y1), None)
    x *= 2.0
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, ptr(x), C.addressof(toks), k, n, ptr(y2), None)
    gncx.check(lib)
    assert np.array_equal(y1, y2)
    assert rel_l2(y1, oracle.matvec(Q4_K, w, x0, k, n)) < TOL
    # without tokens the vector is always re-read
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, ptr(x), None, k, n, ptr(y2), None)
    assert rel_l2(y2, oracle.matvec(Q4_K, w, x, k, n)) < TOL


def test_matvec_device_pointers(lib, oracle):
    """Device-resident x / y / weights: same kernel, same result."""
    torch = pytest.importorskip("torch")
    k, n = 4096, 2048
    w = synth.make_weights(Q4_K, n, k, seed=12)
    x = synth.make_activations(1, k, seed=13)
    wd = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    yd = torch.zeros(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    lib.gncx_xfold_universal_matvec(wd.data_ptr(), 0, Q4_K, xd.data_ptr(), None, k, n, yd.data_ptr(), None)
    assert lib.gncx_hip_synchronize() == 0
    gncx.check(lib)
    yh = np.zeros(n, np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, Q4_K, ptr(x), None, k, n, ptr(yh), None)
    assert np.array_equal(yd.cpu().numpy(), yh)
    assert rel_l2(yh, oracle.matvec(Q4_K, w, x, k, n)) < TOL


# quantised types run on the fp16 matrix cores with fp16-pair operands; cases
# cover every tile size the launcher picks, split K, ragged B and N, and K with
# an odd number of 32-wide steps (k % 64 == 32)
MATBATCH_CASES = [
    (Q4_K, 4096, 512, 64), (Q6_K, 14336, 256, 16), (Q4_0, 4096, 300, 5), (Q8_0, 2048, 200, 9), (Q4_K, 512, 96, 1),
    (BF16, 1024, 64, 4), (Q4_K, 4096, 1024, 256), (Q6_K, 2048, 4160, 100), (Q4_0, 96, 130, 70),
    (Q8_0, 2080, 333, 33),
    (Q4_K, 256, 16384, 300),
    (Q4_K, 256, 8192, 500), (Q6_K, 256, 16384, 128), (Q4_K, 256, 16384, 512), (Q6_K, 512, 8192, 520),
    # the 256-token tiles of 8 waves (256 x 128 and 256 x 64), ragged B and N
    (Q6_K, 256, 24576, 260), (Q4_K, 256, 8192, 300), (Q8_0, 512, 6000, 257),
    # the 8-wave tiles with K split (Q4_K 64 x 256 up to 128 tokens, 128 x 256
    # above; 256 x 128 from 129 tokens for the other types), ragged B and N
    (Q4_K, 2048, 1000, 100), (Q4_K, 4096, 3000, 65), (Q6_K, 4096, 1000, 300), (Q8_0, 2080, 700, 400),
    (Q4_K, 4096, 3000, 200), (Q4_K, 2048, 700, 33),
    # 128 x 128 tiles of 4 waves with K split (65 to 128 tokens, types other than Q4_K)
    (Q8_0, 1024, 640, 128), (Q6_K, 14336, 512, 77),
    # Q4_K at small B: one super-block, K of 3, 5 and 48 super-blocks, ragged B and N
    (Q4_K, 256, 100, 17), (Q4_K, 768, 50, 64), (Q4_K, 1280, 33, 2), (Q4_K, 12288, 200, 48),
    # Q4_K one-product kernel (B >= 1024, whole K): ragged B and N, one and 8 super-blocks
    (Q4_K, 2048, 1000, 1100), (Q4_K, 256, 520, 1030),
    # Q4_K short batches (weights streamed through registers, up to 64 tokens):
    # one and two token tiles, ragged N, K ranges of 1 to 8 super-blocks (the
    # three register sets in turn, ranges of unequal length), one token
    (Q4_K, 12288, 1030, 64), (Q4_K, 20480, 300, 1), (Q4_K, 4096, 777, 40), (Q4_K, 2304, 4100, 63),
    (Q4_K, 4096, 16384, 32), (Q4_K, 2048, 24576, 50), (Q4_K, 3072, 40000, 20), (Q4_K, 1792, 40000, 9),
    (Q4_K, 4096, 6144, 64),
]


@pytest.mark.parametrize("t,k,n,b", MATBATCH_CASES)
def test_matbatch_parity(lib, oracle, t, k, n, b):
    w = synth.make_weights(t, n, k, seed=3000 + t + k + n)
    x = synth.make_activations(b, k, seed=4000 + t + k + n + b).reshape(b, k)
    y = np.full((b, n), np.nan, np.float32)
    lib.gncx_xfold_universal_matbatch(ptr(w), 0, t, ptr(x), b, k, n, ptr(y), None)
    gncx.check(lib)
    err = rel_l2(y, oracle.matbatch(t, w, x, b, k, n))
    print(f"matbatch type={t} k={k} n={n} b={b} rel_l2={err:.3e}")
    assert err < (TOL if t == BF16 else TOL_MATBATCH)


# Q6_K scales beyond +-64 (real quantisers use the whole int8 range): then
# sc (q - 32) can exceed 2048 and the 256-token tiles add the third product in
# the steps that hold such a scale.  All rows large, none, and one row in
# 37 large (single steps of a tile), with K split (k=2048, b=200) and unsplit.
@pytest.mark.parametrize("mode", ["all", "sparse"])
@pytest.mark.parametrize("k,n,b", [(2048, 512, 200), (1024, 3000, 300), (4096, 600, 64), (768, 300, 7)])
def test_matbatch_q6k_large_scales(lib, oracle, mode, k, n, b):
    w = synth.make_weights(Q6_K, n, k, seed=8100 + k + n).reshape(n, k // 256, 210)
    rng = np.random.default_rng(8200 + b)
    big = rng.integers(-128, 128, size=w[..., 192:208].shape).astype(np.int8).view(np.uint8)
    if mode == "all":
        w[..., 192:208] = big
    else:
        rows = np.arange(n) % 37 == 5
        w[rows, :, 192:208] = big[rows]
    w = np.ascontiguousarray(w.reshape(-1))
    x = synth.make_activations(b, k, seed=8300 + b).reshape(b, k)
    y = np.full((b, n), np.nan, np.float32)
    lib.gncx_xfold_universal_matbatch(ptr(w), 0, Q6_K, ptr(x), b, k, n, ptr(y), None)
    gncx.check(lib)
    err = rel_l2(y, oracle.matbatch(Q6_K, w, x, b, k, n))
    print(f"matbatch Q6_K {mode} large scales k={k} n={n} b={b} rel_l2={err:.3e}", flush=True)
    assert err < TOL_MATBATCH


# gncx_hip_swiglu_matbatch: the SwiGLU formed in the activation pass, bit for
# bit the values of gncx_swiglu_activation followed by matbatch; K past the
# quantiser's registers (20480), the one-product Q4_K kernel (B = 1024) and
# BF16 weights (the rows formed first).
@pytest.mark.parametrize("t,k,n,b", [(Q4_K, 4096, 512, 64), (Q4_K, 12288, 256, 300), (Q4_K, 20480, 128, 7),
                                     (Q4_K, 12288, 256, 1024), (Q6_K, 2048, 300, 200), (Q8_0, 1024, 96, 33),
                                     (BF16, 512, 64, 5)])
def test_swiglu_matbatch_equals_two_calls(lib, t, k, n, b):
    w = synth.make_weights(t, n, k, seed=9000 + t + k)
    rng = np.random.default_rng(9100 + b + k)
    gate = (rng.standard_normal((b, k)) * 2).astype(np.float32)
    up = rng.standard_normal((b, k)).astype(np.float32)
    act = np.zeros((b, k), np.float32)
    lib.gncx_swiglu_activation(ptr(gate), ptr(up), b * k, ptr(act))
    want = np.full((b, n), np.nan, np.float32)
    lib.gncx_xfold_universal_matbatch(ptr(w), 0, t, ptr(act), b, k, n, ptr(want), None)
    got = np.full((b, n), np.nan, np.float32)
    try:
        lib.gncx_hip_swiglu_matbatch(ptr(w), 0, t, ptr(gate), ptr(up), b, k, n, ptr(got))
        gncx.check(lib)
    finally:
        lib.gncx_hip_weight_forget(ptr(w))
    assert np.array_equal(got, want)


# The prefill workloads at their own shapes: Q4_K 4096x4096 (Q/O) and
# 4096 -> 14336 (gate/up), Q6_K 14336 -> 4096 (down), at B = 64, 256 and 512,
# plus ragged B past one 256-token tile and the B = 2048 prefill of the
# Qwen3-8B-shaped model (4096 -> 12288 and 12288 -> 4096).
CONFIG3_CASES = [(t, k, n, b) for (t, k, n) in [(Q4_K, 4096, 4096), (Q4_K, 4096, 14336), (Q6_K, 14336, 4096)]
                 for b in (64, 256, 512)] + [
    (Q4_K, 4096, 14336, 300), (Q6_K, 14336, 4096, 511), (Q4_K, 4096, 12288, 2048), (Q4_K, 12288, 4096, 2048)]


@pytest.mark.parametrize("t,k,n,b", CONFIG3_CASES)
def test_matbatch_prefill_shapes(lib, oracle, t, k, n, b):
    w = synth.make_weights(t, n, k, seed=5000 + t + k + n)
    x = synth.make_activations(b, k, seed=6000 + b + k)
    y = np.full((b, n), np.nan, np.float32)
    try:
        lib.gncx_xfold_universal_matbatch(ptr(w), 0, t, ptr(x), b, k, n, ptr(y), None)
        gncx.check(lib)
    finally:
        lib.gncx_hip_weight_forget(ptr(w))
    err = rel_l2(y, oracle.matbatch(t, w, x, b, k, n))
    print(f"matbatch prefill shape type={t} k={k} n={n} b={b} rel_l2={err:.3e}", flush=True)
    assert err < TOL_MATBATCH


# Q/K/V- and gate/up-like groups through gncx_hip_matbatch_multi: the batch is
# quantised once, and the matrices share one launch (and, with split K, one
# reduce) when each is whole 256-row tiles of the plan for their summed rows
# (B = 64 and 100: 64-token tiles, K in 8 ranges; B = 300 and 512:
# 128-token tiles, K in 4 and 2 ranges; B = 2048: no split); otherwise one
# call per matrix (1000 rows: not whole tiles).
MULTI_CASES = [((4096, 1024, 1024), 4096, b) for b in (64, 512, 2048)] + [
    ((1536, 1536), 1024, 300), ((4096, 1000), 2048, 2048), ((256, 512, 256, 1024), 2048, 100)]


@pytest.mark.parametrize("ns,k,b", MULTI_CASES)
def test_matbatch_multi_matches_single_calls(lib, oracle, ns, k, b):
    ws = [synth.make_weights(Q4_K, n, k, seed=7000 + 7 * i + n) for i, n in enumerate(ns)]
    x = synth.make_activations(b, k, seed=7100 + b + k).reshape(b, k)
    ys = [np.full((b, n), np.nan, np.float32) for n in ns]
    P, I = C.c_void_p * len(ns), C.c_int32 * len(ns)
    try:
        lib.gncx_hip_matbatch_multi(len(ns), P(*(w.ctypes.data for w in ws)), I(*ns), Q4_K, ptr(x), b, k,
                                    P(*(y.ctypes.data for y in ys)))
        gncx.check(lib)
        for i, (w, n, y) in enumerate(zip(ws, ns, ys)):
            single = np.full((b, n), np.nan, np.float32)
            lib.gncx_xfold_universal_matbatch(ptr(w), 0, Q4_K, ptr(x), b, k, n, ptr(single), None)
            gncx.check(lib)
            # the same tile arithmetic; a single call that splits K adds its
            # ranges in another order
            assert rel_l2(y, single) < 1e-6
            if b == 2048 and i == 0 and ns[1] % 256 == 0:
                assert np.array_equal(y, single)  # both unsplit 256-row tiles: bit for bit
            err = rel_l2(y, oracle.matbatch(Q4_K, w, x, b, k, n))
            print(f"matbatch multi {ns} k={k} b={b} matrix {i}: rel_l2 {err:.3e}", flush=True)
            assert err < TOL_MATBATCH
    finally:
        for w in ws:
            lib.gncx_hip_weight_forget(ptr(w))


# gncx_hip_matbatch_multi_addnorm against its two steps, add+RMSNorm (or
# RMSNorm alone) into a buffer and gncx_hip_matbatch_multi of it: bit for bit,
# residual rows included.  Q4_K groups of whole 256-row tiles form the norm
# inside the activation pass; (4096, 1000) and Q6_K run the two steps.
ADDNORM_CASES = [(Q4_K, (4096, 1024, 1024), 4096, 64, True), (Q4_K, (4096, 1024, 1024), 4096, 2048, False),
                 (Q4_K, (2048, 2048), 4096, 300, True), (Q4_K, (1536, 512), 5120, 77, True),
                 (Q4_K, (4096, 1000), 2048, 129, True), (Q6_K, (512, 256), 1024, 40, True)]


@pytest.mark.parametrize("t,ns,k,b,add", ADDNORM_CASES)
def test_matbatch_multi_addnorm_matches_two_steps(lib, oracle, torch_mod, t, ns, k, b, add):
    torch = torch_mod
    ws = [synth.make_weights(t, n, k, seed=7300 + 3 * i + n) for i, n in enumerate(ns)]
    rng = np.random.default_rng(7400 + b + k)
    h0 = (rng.standard_normal((b, k)) * 3.0).astype(np.float32)
    d0 = rng.standard_normal((b, k)).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    eps = 1e-6
    dev = lambda a: torch.from_numpy(a).cuda()
    h1, h2, dd = dev(h0), dev(h0), dev(d0)
    xn = torch.zeros(b, k, dtype=torch.float32, device="cuda")
    y1 = [torch.full((b, n), float("nan"), device="cuda") for n in ns]
    y2 = [torch.full((b, n), float("nan"), device="cuda") for n in ns]
    P, I = C.c_void_p * len(ns), C.c_int32 * len(ns)
    wp = P(*(w.ctypes.data for w in ws))
    torch.cuda.synchronize()
    print(f"matbatch multi addnorm type={t} {ns} k={k} b={b} add={add}", flush=True)
    try:
        lib.gncx_hip_matbatch_multi_addnorm(h1.data_ptr(), dd.data_ptr() if add else None, gamma.ctypes.data, 0,
                                            eps, len(ns), wp, I(*ns), t, b, k, P(*(y.data_ptr() for y in y1)))
        gncx.check(lib)
        if add:
            lib.gncx_hip_add_rmsnorm_rows(h2.data_ptr(), dd.data_ptr(), b, gamma.ctypes.data, 0, k, eps,
                                          xn.data_ptr())
        else:
            lib.gncx_hip_rmsnorm_rows(h2.data_ptr(), b, gamma.ctypes.data, 0, k, eps, xn.data_ptr())
        gncx.check(lib)
        lib.gncx_hip_matbatch_multi(len(ns), wp, I(*ns), t, xn.data_ptr(), b, k, P(*(y.data_ptr() for y in y2)))
        gncx.check(lib)
        assert lib.gncx_hip_synchronize() == 0
    finally:
        for w in ws:
            lib.gncx_hip_weight_forget(ptr(w))
    assert torch.equal(h1, h2)
    assert np.array_equal(h1.cpu().numpy(), h0 + d0 if add else h0)
    x = xn.cpu().numpy()
    for w, n, a, c in zip(ws, ns, y1, y2):
        a, c = a.cpu().numpy(), c.cpu().numpy()
        assert np.array_equal(a, c)
        assert rel_l2(a, oracle.matbatch(t, w, x, b, k, n)) < TOL_MATBATCH


def test_matbatch_multi_addnorm_rejects_host_rows(lib, torch_mod):
    """hidden, delta and the outputs must be device memory: host rows are
    refused with an error before anything runs, and the host rows stay as
    they were."""
    torch = torch_mod
    k, b, ns = 256, 4, (256, 256)
    ws = [synth.make_weights(Q4_K, n, k, seed=7500 + n + i) for i, n in enumerate(ns)]
    gamma = np.ones(k, np.float32)
    h = np.arange(b * k, dtype=np.float32)
    ys = [torch.zeros(b, n, device="cuda") for n in ns]
    P, I = C.c_void_p * 2, C.c_int32 * 2
    torch.cuda.synchronize()
    lib.gncx_hip_matbatch_multi_addnorm(h.ctypes.data, None, gamma.ctypes.data, 0, 1e-6, 2,
                                        P(*(w.ctypes.data for w in ws)), I(*ns), Q4_K, b, k,
                                        P(*(y.data_ptr() for y in ys)))
    with pytest.raises(RuntimeError, match="device memory"):
        gncx.check(lib)
    assert np.array_equal(h, np.arange(b * k, dtype=np.float32))
    for w in ws:
        lib.gncx_hip_weight_forget(ptr(w))


def test_lm_head_and_softcap(lib, golden):
    w, x = golden["lm_w"].copy(), golden["lm_x"].copy()
    v, k = int(golden["lm_vocab"]), int(golden["lm_k"])
    y = np.zeros(v, np.float32)
    lib.gncx_universal_lm_head_logits(ptr(w), 0, Q6_K, ptr(x), k, v, 0.0, ptr(y))
    gncx.check(lib)
    assert rel_l2(y, golden["lm_y"]) < TOL
    lib.gncx_universal_lm_head_logits(ptr(w), 0, Q6_K, ptr(x), k, v, 30.0, ptr(y))
    gncx.check(lib)
    assert rel_l2(y, golden["lm_y_cap"]) < TOL


MULTI_CASES = [
    # (type, k, out_dims): Q/K/V and gate/up of the Qwen3-8B-shaped model, other types,
    # a K-split shape, and one the band kernel does not take (one launch per matrix)
    (Q4_K, 4096, (4096, 1024, 1024)),
    (Q4_K, 4096, (12288, 12288)),
    (Q4_K, 14336, (4096, 33)),
    (Q6_K, 4096, (300, 1, 77, 4096)),
    (Q8_0, 4096, (1024, 512)),
    (Q4_0, 2048, (5, 700)),
    (BF16, 1024, (256, 128, 64)),
    (Q4_0, 40960, (8, 3)),
]


@pytest.mark.parametrize("t,k,dims", MULTI_CASES)
def test_matvec_multi_equals_separate_matvecs(lib, t, k, dims):
    """gncx_hip_matvec_multi: each output bit-identical to the same matrix's
    gncx_xfold_universal_matvec (every row's dot runs the same arithmetic)."""
    ws = [synth.make_weights(t, n, k, seed=300 + i + t) for i, n in enumerate(dims)]
    x = synth.make_activations(1, k, seed=400 + t + k)
    want = []
    for w, n in zip(ws, dims):
        y = np.full(n, np.nan, np.float32)
        lib.gncx_xfold_universal_matvec(ptr(w), 0, t, ptr(x), None, k, n, ptr(y), None)
        gncx.check(lib)
        want.append(y)
    outs = [np.full(n, np.nan, np.float32) for n in dims]
    cnt = len(dims)
    lib.gncx_hip_matvec_multi(cnt, (C.c_void_p * cnt)(*[ptr(w) for w in ws]), (C.c_int32 * cnt)(*dims), t, ptr(x),
                              k, (C.c_void_p * cnt)(*[ptr(o) for o in outs]))
    gncx.check(lib)
    for i, (got, w) in enumerate(zip(outs, want)):
        assert np.array_equal(got, w), (i, float(np.abs(got - w).max()))
    for w in ws:
        lib.gncx_hip_weight_forget(ptr(w))


def test_matvec_multi_rejects_bad_counts(lib):
    x = np.zeros(256, np.float32)
    y = np.zeros(8, np.float32)
    w = synth.make_weights(Q4_K, 8, 256, seed=1)
    for cnt in (0, 5):
        lib.gncx_hip_matvec_multi(cnt, (C.c_void_p * 5)(*[ptr(w)] * 5), (C.c_int32 * 5)(*[8] * 5), Q4_K, ptr(x), 256,
                                  (C.c_void_p * 5)(*[ptr(y)] * 5))
        assert lib.gncx_hip_last_status() != 0
    lib.gncx_hip_weight_forget(ptr(w))


@pytest.mark.parametrize("t,k,ns,with_delta", [
    (gncx.Q4_K, 4096, (4096, 1024, 1024), True),
    (gncx.Q4_K, 4096, (12288, 12288), True),
    (gncx.Q8_0, 2048, (512, 256, 256), False),
    (gncx.Q6_K, 1024, (300,), True),
    (gncx.Q4_0, 4096, (64,), True),
    (gncx.Q8_0, 4096, (1024,), True),
])
def test_matvec_multi_addnorm_equals_separate_calls(lib, torch_mod, t, k, ns, with_delta):
    """Residual add + RMSNorm formed inside the matvec launch: outputs and the
    new residual equal gncx_hip_add_rmsnorm followed by gncx_hip_matvec_multi
    bit for bit.  Q8_0 at k = 4096 needs two K-slices per row, which the fused
    schedule does not take: the call runs the separate kernels instead."""
    torch = torch_mod
    P, I = C.c_void_p, C.c_int32
    ws = [torch.from_numpy(synth.make_weights(t, n, k, seed=40 + i)).cuda() for i, n in enumerate(ns)]
    g = torch.Generator(device="cuda").manual_seed(3)
    h = torch.randn(k, device="cuda", generator=g)
    r = torch.randn(k, device="cuda", generator=g) if with_delta else None
    gamma = 1.0 + 0.1 * torch.randn(k, device="cuda", generator=g)
    h_out = torch.zeros(k, device="cuda")
    ys = [torch.zeros(n, device="cuda") for n in ns]
    cnt = len(ns)
    wa = (P * cnt)(*(w.data_ptr() for w in ws))
    na = (I * cnt)(*ns)
    ya = (P * cnt)(*(y.data_ptr() for y in ys))
    lib.gncx_hip_matvec_multi_addnorm(h.data_ptr(), r.data_ptr() if r is not None else None, gamma.data_ptr(), 0,
                                      1e-6, h_out.data_ptr(), cnt, wa, na, t, k, ya)
    gncx.check(lib)
    # the separate calls
    h2 = h.clone()
    normed = torch.zeros(k, device="cuda")
    if r is not None:
        lib.gncx_hip_add_rmsnorm(h2.data_ptr(), r.data_ptr(), gamma.data_ptr(), 0, k, 1e-6, normed.data_ptr())
    else:
        lib.gncx_rmsnorm_and_encode_4phase(h2.data_ptr(), gamma.data_ptr(), 0, k, 1e-6, 0, normed.data_ptr(), None,
                                           None)
    ys2 = [torch.zeros(n, device="cuda") for n in ns]
    lib.gncx_hip_matvec_multi(cnt, wa, na, t, normed.data_ptr(), k, (P * cnt)(*(y.data_ptr() for y in ys2)))
    gncx.check(lib)
    torch.cuda.synchronize()
    for a, b in zip(ys, ys2):
        assert torch.equal(a, b), (a - b).abs().max().item()
    if r is not None:
        assert torch.equal(h_out, h2)
    else:
        assert torch.equal(h_out, h)


@pytest.mark.parametrize("t,k,f", [(gncx.Q4_K, 4096, 12288), (gncx.Q4_K, 1024, 512), (gncx.Q8_0, 512, 96),
                                   (gncx.Q6_K, 4096, 1024)])
def test_matvec_swiglu_equals_separate_calls(lib, torch_mod, t, k, f):
    """gate/up matvecs with SiLU(gate) * up in the launch's epilogue equal two
    matvecs and gncx_swiglu_activation bit for bit (f = 96 with Q8_0 does not
    split over the grid and takes the separate kernels)."""
    torch = torch_mod
    wg = torch.from_numpy(synth.make_weights(t, f, k, seed=51)).cuda()
    wu = torch.from_numpy(synth.make_weights(t, f, k, seed=52)).cuda()
    x = torch.from_numpy(synth.make_activations(1, k, seed=53)).cuda()
    act = torch.zeros(f, device="cuda")
    lib.gncx_hip_matvec_swiglu(wg.data_ptr(), wu.data_ptr(), t, x.data_ptr(), k, f, act.data_ptr())
    gncx.check(lib)
    gate = torch.zeros(f, device="cuda")
    up = torch.zeros(f, device="cuda")
    want = torch.zeros(f, device="cuda")
    lib.gncx_xfold_universal_matvec(wg.data_ptr(), 0, t, x.data_ptr(), None, k, f, gate.data_ptr(), None)
    lib.gncx_xfold_universal_matvec(wu.data_ptr(), 0, t, x.data_ptr(), None, k, f, up.data_ptr(), None)
    lib.gncx_swiglu_activation(gate.data_ptr(), up.data_ptr(), f, want.data_ptr())
    gncx.check(lib)
    torch.cuda.synchronize()
    assert torch.equal(act, want), (act - want).abs().max().item()
