"""GPU parity of the decode-attention step and its prologue, through the
C-ABI: gncx_mqa_attention_step_ext against the oracle (1e-3 relative L2 bar;
observed ~1e-7), KV-cache write-back into host caches, multi-step decode
through one host cache, the fused norm+RoPE+attention entry against the
reference call sequence, and the per-head RMSNorm / RoPE / SwiGLU / RMSNorm /
embedding companions."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import synth
from conftest import gncx, ptr, rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3


def run_attention(lib, q, kn, vn, kc, vc, pos, H, KV, hd, scale, sw, write_kv):
    out = np.full(H * hd, np.nan, np.float32)
    lib.gncx_mqa_attention_step_ext(ptr(q), ptr(kn), ptr(vn), ptr(kc), ptr(vc), pos, H, KV, hd, scale, sw,
                                    write_kv, ptr(out))
    gncx.check(lib)
    return out


@pytest.mark.parametrize("tag", ["gqa", "swa", "mqa"])
def test_attention_reference_vectors(lib, golden, tag):
    g = golden
    pos, H, kv, hd, sw = (int(v) for v in g[f"attn_{tag}_geom"])
    kc, vc = g[f"attn_{tag}_kc"].copy(), g[f"attn_{tag}_vc"].copy()
    kn, vn = g[f"attn_{tag}_kn"].copy(), g[f"attn_{tag}_vn"].copy()
    out = run_attention(lib, g[f"attn_{tag}_q"].copy(), kn, vn, kc, vc, pos, H, kv, hd, 1 / np.sqrt(hd), sw, 1)
    assert rel_l2(out, g[f"attn_{tag}_out"]) < TOL
    # the new row was written into the caller's (host) cache
    assert np.array_equal(kc[pos], kn) and np.array_equal(vc[pos], vn)
    lib.gncx_hip_kv_forget(None)


# config 4: 32 Q / 8 KV heads x 128, ctx 512 / 4096 / 32768, SWA 1024, MQA
CASES = [(32, 8, 128, 512, 0), (32, 8, 128, 4096, 0), (32, 8, 128, 32768, 0), (32, 8, 128, 4096, 1024),
         (32, 8, 128, 32768, 1024), (32, 1, 128, 512, 0), (32, 1, 128, 4096, 0), (32, 1, 128, 32768, 0),
         (16, 16, 64, 300, 0),
         (8, 2, 256, 700, 100), (4, 4, 128, 1, 0),
         # query-head groups of 16..32 (matrix-core kernel): one token, ragged
         # sliding window, 16 heads padded to 32, two KV heads, partial sub-chunk
         (32, 1, 128, 1, 0), (32, 1, 128, 100, 50), (16, 1, 128, 333, 0), (64, 2, 128, 2000, 0),
         (32, 2, 128, 129, 0),
         # windows past 32-token chunks at 1024 work-groups: longer chunks,
         # ragged (the last chunk partial), 4 KV heads, a sliding window
         (32, 8, 128, 8193, 0), (32, 4, 128, 20000, 0), (32, 8, 128, 20000, 6000)]


@pytest.mark.parametrize("H,KV,hd,ctx,sw", CASES)
def test_attention_parity(lib, oracle, H, KV, hd, ctx, sw):
    rng = np.random.default_rng(H * 1000 + KV * 100 + ctx + sw)
    kc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    vc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    q = rng.standard_normal(H * hd, dtype=np.float32)
    kn = rng.standard_normal(KV * hd, dtype=np.float32)
    vn = rng.standard_normal(KV * hd, dtype=np.float32)
    pos = ctx - 1
    want, kc_w, vc_w = oracle.attention(q, kn, vn, kc, vc, pos, H, KV, hd, 1 / np.sqrt(hd), sw, 1)
    out = run_attention(lib, q, kn, vn, kc, vc, pos, H, KV, hd, 1 / np.sqrt(hd), sw, 1)
    err = rel_l2(out, want)
    print(f"attention H={H} KV={KV} hd={hd} ctx={ctx} sw={sw} rel_l2={err:.3e}")
    assert err < TOL
    assert np.array_equal(kc, kc_w) and np.array_equal(vc, vc_w)
    lib.gncx_hip_kv_forget(None)


@pytest.mark.parametrize("H,KV", [(8, 2), (32, 1)])
def test_attention_write_kv_off_uses_cached_row(lib, oracle, H, KV):
    rng = np.random.default_rng(3)
    hd, ctx = 128, 64
    kc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    vc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    q = rng.standard_normal(H * hd, dtype=np.float32)
    kn = rng.standard_normal(KV * hd, dtype=np.float32)
    want, _, _ = oracle.attention(q, kn, kn, kc, vc, 40, H, KV, hd, 0.1, 0, 0)
    kc0 = kc.copy()
    out = run_attention(lib, q, kn, kn, kc, vc, 40, H, KV, hd, 0.1, 0, 0)
    assert rel_l2(out, want) < TOL
    assert np.array_equal(kc, kc0)
    lib.gncx_hip_kv_forget(None)


def test_decode_sequence_through_one_host_cache(lib, oracle):
    """60 steps pos = 0..59 into the same host caches, as the streamer does;
    the device twin stays coherent with the host rows."""
    rng = np.random.default_rng(4)
    H, KV, hd, rows = 16, 4, 128, 64
    kc = np.zeros((rows, KV * hd), np.float32)
    vc = np.zeros((rows, KV * hd), np.float32)
    okc, ovc = kc.copy(), vc.copy()
    worst = 0.0
    for pos in range(60):
        q = rng.standard_normal(H * hd, dtype=np.float32)
        kn = rng.standard_normal(KV * hd, dtype=np.float32)
        vn = rng.standard_normal(KV * hd, dtype=np.float32)
        sw = 16 if pos % 3 == 0 else 0
        want, okc, ovc = oracle.attention(q, kn, vn, okc, ovc, pos, H, KV, hd, 0.0884, sw, 1)
        out = run_attention(lib, q, kn, vn, kc, vc, pos, H, KV, hd, 0.0884, sw, 1)
        worst = max(worst, rel_l2(out, want))
    assert worst < TOL
    assert np.array_equal(kc, okc) and np.array_equal(vc, ovc)
    lib.gncx_hip_kv_forget(None)


def test_kv_twin_notices_rewritten_host_cache(lib, oracle):
    rng = np.random.default_rng(5)
    H, KV, hd, ctx = 8, 8, 64, 50
    kc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    vc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    q = rng.standard_normal(H * hd, dtype=np.float32)
    run_attention(lib, q, kc[30], vc[30], kc, vc, 30, H, KV, hd, 0.125, 0, 1)
    kc[:] = rng.standard_normal((ctx, KV * hd), dtype=np.float32)  # caller refills the cache
    vc[:] = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    want, _, _ = oracle.attention(q, None, None, kc, vc, 20, H, KV, hd, 0.125, 0, 0)
    out = run_attention(lib, q, None, None, kc, vc, 20, H, KV, hd, 0.125, 0, 0)
    assert rel_l2(out, want) < TOL
    lib.gncx_hip_kv_forget(None)


@pytest.mark.parametrize("H,KV,hd,ctx,sw", [(32, 8, 128, 4096, 0), (32, 1, 128, 600, 0), (8, 4, 64, 300, 128)])
def test_fused_prologue_equals_reference_sequence(lib, oracle, H, KV, hd, ctx, sw):
    """gncx_hip_attention_step_fused == rmsnorm_heads(q), rmsnorm_heads(k),
    rope(q, k), attention_step -- on the GPU and against the oracle."""
    rng = np.random.default_rng(ctx + H)
    kc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    vc = rng.standard_normal((ctx, KV * hd), dtype=np.float32)
    q = rng.standard_normal(H * hd, dtype=np.float32)
    kn = rng.standard_normal(KV * hd, dtype=np.float32)
    vn = rng.standard_normal(KV * hd, dtype=np.float32)
    gq, gk = synth.make_norm_gamma(hd, 1), synth.make_norm_gamma(hd, 2)
    norms = np.concatenate([gq, gk]).astype(np.float32)
    pos, eps, base, scale = ctx - 1, 1e-6, 1e6, 1 / np.sqrt(hd)

    # oracle sequence
    oq = oracle.rmsnorm_heads(q, gq, H, hd, eps)
    ok = oracle.rmsnorm_heads(kn, gk, KV, hd, eps)
    oq, ok = oracle.rope(oq, ok, H, KV, hd, pos, base)
    want, owk, _ = oracle.attention(oq, ok, vn, kc, vc, pos, H, KV, hd, scale, sw, 1)

    # library, step by step (the streamer's calls, streamer.lua:817-862)
    q1, k1, kc1, vc1 = q.copy(), kn.copy(), kc.copy(), vc.copy()
    lib.gncx_rmsnorm_inplace_heads(ptr(q1), ptr(norms), 0, 1, H, hd, eps)
    lib.gncx_rmsnorm_inplace_heads(ptr(k1), ptr(norms), hd * 4, 1, KV, hd, eps)
    lib.gncx_apply_rope_xor11_ext(ptr(q1), ptr(k1), None, None, 0, 0, H, KV, hd, pos, base)
    out1 = run_attention(lib, q1, k1, vn, kc1, vc1, pos, H, KV, hd, scale, sw, 1)
    lib.gncx_hip_kv_forget(None)

    # library, fused
    q2, k2, kc2, vc2 = q.copy(), kn.copy(), kc.copy(), vc.copy()
    out2 = np.zeros(H * hd, np.float32)
    lib.gncx_hip_attention_step_fused(ptr(q2), ptr(k2), ptr(vn), ptr(kc2), ptr(vc2), pos, H, KV, hd, scale, sw, 1,
                                      ptr(norms), 0, hd * 4, 1, eps, 0, 0, base, ptr(out2))
    gncx.check(lib)
    lib.gncx_hip_kv_forget(None)

    assert np.array_equal(q1, q2) and np.array_equal(k1, k2)
    assert np.array_equal(kc1, kc2)
    assert rel_l2(out2, out1) < 1e-6
    assert rel_l2(q1, oq) < 1e-6 and rel_l2(k1, ok) < 1e-6
    assert rel_l2(out2, want) < TOL
    assert rel_l2(kc2[pos], owk[pos]) < 1e-6


def test_rmsnorm_heads_and_rope_vectors(lib, golden):
    v = golden["rmsh_v"].copy()
    g = golden["rmsh_g"].copy()
    lib.gncx_rmsnorm_inplace_heads(ptr(v), ptr(g), 0, 1, 8, 128, 1e-6)
    gncx.check(lib)
    assert rel_l2(v, golden["rmsh_y"]) < 1e-6
    v = golden["rmsh_v"].copy()
    lib.gncx_rmsnorm_inplace_heads(ptr(v), None, 0, 0, 8, 128, 1e-6)
    assert rel_l2(v, golden["rmsh_y_nog"]) < 1e-6
    for p in (0, 1, 511, 4095, 32767):
        q, k = golden["rope_q"].copy(), golden["rope_k"].copy()
        lib.gncx_apply_rope_xor11_ext(ptr(q), ptr(k), None, None, 0, 0, 4, 2, 128, p, 1e6)
        gncx.check(lib)
        assert rel_l2(q, golden[f"rope_q_{p}"]) < 1e-6 and rel_l2(k, golden[f"rope_k_{p}"]) < 1e-6
    q, k, f = golden["rope_q"].copy(), golden["rope_k"].copy(), golden["rope_f"].copy()
    lib.gncx_apply_rope_xor11_ext(ptr(q), ptr(k), None, ptr(f), 0, 1, 4, 2, 128, 777, 1e4)
    assert rel_l2(q, golden["rope_q_fac"]) < 1e-6 and rel_l2(k, golden["rope_k_fac"]) < 1e-6


def test_rmsnorm_heads_bitexact_with_oracle(lib, oracle):
    rng = np.random.default_rng(9)
    v = rng.standard_normal(32 * 128, dtype=np.float32)
    g = synth.make_norm_gamma(128, 3)
    out = v.copy()
    lib.gncx_rmsnorm_inplace_heads(ptr(out), ptr(g), 0, 1, 32, 128, 1e-6)
    gncx.check(lib)
    assert np.array_equal(out, oracle.rmsnorm_heads(v, g, 32, 128, 1e-6))


@pytest.mark.parametrize("dim", [4096, 4098, 12288, 20000, 40960, 7])
def test_rmsnorm_shapes(lib, oracle, dim):
    """float4 path (registers, and the loop past 16384 values), scalar tail
    and scalar-only rows"""
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 3).astype(np.float32)
    g = synth.make_norm_gamma(dim, dim + 1)
    out = np.zeros_like(x)
    lib.gncx_rmsnorm_and_encode_4phase(ptr(x), ptr(g), 0, dim, 1e-6, 0, ptr(out), None, None)
    gncx.check(lib)
    assert rel_l2(out, oracle.rmsnorm(x, g, 1e-6)) < 1e-6


@pytest.mark.parametrize("dim", [4096, 4098, 20000, 7])
def test_add_rmsnorm_equals_vec_add_then_rmsnorm(lib, oracle, dim):
    """gncx_hip_add_rmsnorm = gncx_hip_vec_add then gncx_rmsnorm_and_encode_4phase,
    bit for bit, for the new hidden and the normalised output (host buffers)."""
    rng = np.random.default_rng(dim + 5)
    h0 = (rng.standard_normal(dim) * 3).astype(np.float32)
    d = rng.standard_normal(dim).astype(np.float32)
    g = synth.make_norm_gamma(dim, dim + 2)
    h1 = h0.copy()
    lib.gncx_hip_vec_add(ptr(h1), ptr(d), dim)
    want = np.zeros_like(h0)
    lib.gncx_rmsnorm_and_encode_4phase(ptr(h1), ptr(g), 0, dim, 1e-6, 0, ptr(want), None, None)
    gncx.check(lib)
    h2 = h0.copy()
    got = np.zeros_like(h0)
    lib.gncx_hip_add_rmsnorm(ptr(h2), ptr(d), ptr(g), 0, dim, 1e-6, ptr(got))
    gncx.check(lib)
    assert np.array_equal(h2, h1)
    assert np.array_equal(h2, h0 + d)
    assert np.array_equal(got, want)
    assert rel_l2(got, oracle.rmsnorm(h0 + d, g, 1e-6)) < 1e-6


@pytest.mark.parametrize("n_heads,hd", [(1, 4096), (3, 640), (5, 512), (2, 96)])
def test_rmsnorm_heads_long_and_odd_heads_bitexact(lib, oracle, n_heads, hd):
    rng = np.random.default_rng(n_heads * hd)
    v = rng.standard_normal(n_heads * hd, dtype=np.float32)
    g = synth.make_norm_gamma(hd, 7)
    out = v.copy()
    lib.gncx_rmsnorm_inplace_heads(ptr(out), ptr(g), 0, 1, n_heads, hd, 1e-6)
    gncx.check(lib)
    assert np.array_equal(out, oracle.rmsnorm_heads(v, g, n_heads, hd, 1e-6))


def test_rmsnorm_swiglu_embeddings(lib, golden, oracle):
    x, g = golden["rms_x"].copy(), golden["rms_g"].copy()
    out = np.zeros_like(x)
    lib.gncx_rmsnorm_and_encode_4phase(ptr(x), ptr(g), 0, x.size, 1e-6, 0, ptr(out), None, None)
    gncx.check(lib)
    assert rel_l2(out, golden["rms_y"]) < 1e-6
    gg, uu = golden["swi_g"].copy(), golden["swi_u"].copy()
    o = np.zeros_like(gg)
    lib.gncx_swiglu_activation(ptr(gg), ptr(uu), gg.size, ptr(o))
    gncx.check(lib)
    assert rel_l2(o, golden["swi_y"]) < 1e-6
    for name, fn in (("q8_0", lib.gncx_fetch_token_embedding_q8_0), ("q6_k", lib.gncx_fetch_token_embedding_q6_k),
                     ("bf16", lib.gncx_fetch_token_embedding_bf16)):
        tab = golden[f"emb_{name}_tab"].copy()
        e = np.zeros(512, np.float32)
        fn(ptr(tab), 0, 5, 512, 1.0, ptr(e))
        gncx.check(lib)
        assert np.array_equal(e, golden[f"emb_{name}_y5"])
        fn(ptr(tab), 0, 11, 512, 0.37, ptr(e))
        assert np.array_equal(e, golden[f"emb_{name}_y11s"])


@pytest.mark.parametrize("name,t", [("q8_0", 8), ("q6_k", 14), ("bf16", 30)])
def test_fetch_token_embeddings_rows(lib, golden, name, t):
    """gncx_hip_fetch_token_embeddings equals one per-token fetch per row, bit
    for bit (and the golden rows); an id outside the table is refused on the
    host, before anything is launched."""
    fn = {8: lib.gncx_fetch_token_embedding_q8_0, 14: lib.gncx_fetch_token_embedding_q6_k,
          30: lib.gncx_fetch_token_embedding_bf16}[t]
    tab, dim = golden[f"emb_{name}_tab"].copy(), 512
    vocab = tab.nbytes // gncx.row_bytes(t, dim)
    ids = np.array([5, 0, vocab - 1, 11, 5, 3], np.int32)
    out = np.full((len(ids), dim), np.nan, np.float32)
    lib.gncx_hip_fetch_token_embeddings(t, ptr(tab), 0, ptr(ids), len(ids), vocab, dim, 0.37, ptr(out))
    gncx.check(lib)
    for i, tok in enumerate(ids):
        e = np.zeros(dim, np.float32)
        fn(ptr(tab), 0, int(tok), dim, 0.37, ptr(e))
        gncx.check(lib)
        assert np.array_equal(out[i], e)
    assert np.array_equal(out[3], golden[f"emb_{name}_y11s"])
    bad = np.array([1, vocab], np.int32)
    before = out.copy()
    lib.gncx_hip_fetch_token_embeddings(t, ptr(tab), 0, ptr(bad), 2, vocab, dim, 1.0, ptr(out))
    assert lib.gncx_hip_last_status() != 0
    assert np.array_equal(out, before)
    lib.gncx_hip_weight_forget(ptr(tab))


@pytest.mark.parametrize("lk", [0, 2, 3, 9, 17])
def test_rmsnorm_encode_tokens_bitexact(lib, golden, lk):
    """The 4-phase encode runs on the device: its tokens and quant scale equal
    the reference's bit for bit, for host and for device outputs."""
    x, g = golden["rms_x"].copy(), golden["rms_g"].copy()
    out = np.zeros_like(x)
    tok = (gncx.GNCXCompactToken * x.size)()
    qs = np.zeros(1, np.float32)
    lib.gncx_rmsnorm_and_encode_4phase(ptr(x), ptr(g), 0, x.size, 1e-6, lk, ptr(out), C.addressof(tok), ptr(qs))
    gncx.check(lib)
    got = np.frombuffer(bytes(tok), dtype=np.uint32)
    assert np.array_equal(got, golden[f"enc_tok_k{lk}"])
    assert qs[0] == golden[f"enc_qs_k{lk}"]
    assert rel_l2(out, golden["rms_y"]) < 1e-6


def _cancellations(tok):
    """sum over digits d of min(#tokens with value >= 0, #tokens below 0)."""
    d, pos = (tok >> 8) & 0xFF, (tok >> 1) & 1
    return sum(min(int(np.sum((d == i) & (pos == 1))), int(np.sum((d == i) & (pos == 0)))) for i in range(10))


@pytest.mark.parametrize("dim,lk", [(4096, 0), (4096, 3), (12288, 2), (16384, 1), (4098, 2), (20000, 0), (100, 9)])
def test_rmsnorm_encode_paths_and_cancellations(lib, oracle, dim, lk):
    """Both encode paths -- the row held in registers (dim a multiple of 4 up
    to 16384) and the second pass over the stored row (other dims) -- give
    the oracle's tokens and scale for the normed vector, and the cancellation
    count the device forms reaches the telemetry of a matvec on those tokens
    (cpp:882-887, cpp:1464-1470)."""
    rng = np.random.default_rng(dim + lk)
    x = rng.standard_normal(dim).astype(np.float32)
    x[rng.integers(0, dim, 5)] *= 40.0
    g = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    out = np.zeros_like(x)
    tok = (gncx.GNCXCompactToken * dim)()
    qs = np.zeros(1, np.float32)
    lib.gncx_rmsnorm_and_encode_4phase(ptr(x), ptr(g), 0, dim, 1e-6, lk, ptr(out), C.addressof(tok), ptr(qs))
    gncx.check(lib)
    got = np.frombuffer(bytes(tok), dtype=np.uint32).copy()
    want, want_qs = oracle.encode(out, lk)
    assert np.array_equal(got, want)
    assert qs[0] == want_qs
    # the encode's own tokens: the count is the one formed with them
    k, n = 256, 8
    w = synth.make_weights(12, n, k, seed=dim)
    xk = synth.make_activations(1, k, seed=lk)
    y = np.zeros(n, np.float32)
    tel = gncx.GNCXTelemetryStats()
    lib.gncx_xfold_universal_matvec(ptr(w), 0, 12, ptr(xk), C.addressof(tok), k, n, ptr(y), C.addressof(tel))
    gncx.check(lib)
    assert tel.zero_origin_cancellations == _cancellations(want) > 0


PREFILL_CASES = [
    # (H, KV, hd, pos0, B, sw): fresh prompt, a cache prefix, a sliding window,
    # MQA (32 heads on one KV head), one head per KV head, and a head_dim the
    # batched kernels do not take (one fused step per token inside the call)
    (32, 8, 128, 0, 100, 0),
    (32, 8, 128, 37, 70, 0),
    (32, 8, 128, 5, 50, 16),
    (32, 1, 128, 3, 20, 0),
    (16, 16, 128, 0, 40, 0),
    (8, 2, 64, 2, 10, 0),
    # key ranges of more than 8 sub-chunks of 32 keys: the longer blocks are
    # cut into up to three work-groups whose parts a merge kernel combines --
    # a fresh prompt, a cache prefix (every block cut), a sliding window, MQA,
    # and one head per KV head (128-token blocks)
    (32, 8, 128, 0, 600, 0),
    (32, 8, 128, 500, 100, 0),
    (32, 8, 128, 0, 700, 300),
    (32, 1, 128, 0, 400, 0),
    (16, 16, 128, 3, 520, 0),
]


def _prefill_inputs(H, KV, hd, pos0, B, seed):
    rng = np.random.default_rng(seed)
    rows = pos0 + B
    kc = np.zeros((rows, KV * hd), np.float32)
    vc = np.zeros((rows, KV * hd), np.float32)
    kc[:pos0] = rng.standard_normal((pos0, KV * hd), dtype=np.float32)
    vc[:pos0] = rng.standard_normal((pos0, KV * hd), dtype=np.float32)
    q = rng.standard_normal((B, H * hd), dtype=np.float32)
    k = rng.standard_normal((B, KV * hd), dtype=np.float32)
    v = rng.standard_normal((B, KV * hd), dtype=np.float32)
    norms = np.concatenate([synth.make_norm_gamma(hd, 3), synth.make_norm_gamma(hd, 4)]).astype(np.float32)
    return kc, vc, q, k, v, norms


@pytest.mark.parametrize("H,KV,hd,pos0,B,sw", PREFILL_CASES)
def test_attention_prefill_equals_fused_steps(lib, H, KV, hd, pos0, B, sw):
    """gncx_hip_attention_prefill == gncx_hip_attention_step_fused per token in
    turn (host buffers): q/k prologue results and the new cache rows bit for
    bit, outputs within 1e-5 (online softmax against split-K plus merge)."""
    kc, vc, q, k, v, norms = _prefill_inputs(H, KV, hd, pos0, B, H * 1000 + B + pos0)
    eps, base, scale = 1e-6, 1e6, 1 / np.sqrt(hd)
    q1, k1, kc1, vc1 = q.copy(), k.copy(), kc.copy(), vc.copy()
    out1 = np.zeros((B, H * hd), np.float32)
    for t in range(B):
        lib.gncx_hip_attention_step_fused(ptr(q1[t]), ptr(k1[t]), ptr(v[t]), ptr(kc1), ptr(vc1), pos0 + t, H, KV, hd,
                                          scale, sw, 1, ptr(norms), 0, hd * 4, 1, eps, 0, 0, base, ptr(out1[t]))
    gncx.check(lib)
    lib.gncx_hip_kv_forget(None)
    q2, k2, kc2, vc2 = q.copy(), k.copy(), kc.copy(), vc.copy()
    out2 = np.zeros((B, H * hd), np.float32)
    lib.gncx_hip_attention_prefill(ptr(q2), ptr(k2), ptr(v), ptr(kc2), ptr(vc2), pos0, B, H, KV, hd, scale, sw,
                                   ptr(norms), 0, hd * 4, 1, eps, 0, 0, base, ptr(out2))
    gncx.check(lib)
    lib.gncx_hip_kv_forget(None)
    assert np.array_equal(q1, q2) and np.array_equal(k1, k2)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
    errs = [rel_l2(out2[t], out1[t]) for t in range(B)]
    print(f"prefill H={H} KV={KV} hd={hd} pos0={pos0} B={B} sw={sw} max row rel_l2={max(errs):.2e}")
    assert max(errs) < 1e-5


@pytest.mark.parametrize("pos0,B,sw", [(10, 64, 0), (300, 200, 0), (0, 600, 200)])
def test_attention_prefill_device_buffers(lib, oracle, pos0, B, sw):
    """Device-resident buffers (used in place), against the oracle's
    per-token prologue followed by its batched causal attention.  The second
    and third shapes run the key-split plan (a cache prefix; a sliding window
    over a fresh prompt), so the parts' merge is checked against the oracle
    directly."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    H, KV, hd = 32, 8, 128
    kc, vc, q, k, v, norms = _prefill_inputs(H, KV, hd, pos0, B, 99 + pos0 + B)
    eps, base, scale = 1e-6, 1e6, 1 / np.sqrt(hd)
    gq, gk = norms[:hd], norms[hd:]
    okc, ovc = kc.copy(), vc.copy()
    oqs = np.zeros((B, H * hd), np.float32)
    for t in range(B):
        oq = oracle.rmsnorm_heads(q[t], gq, H, hd, eps)
        ok = oracle.rmsnorm_heads(k[t], gk, KV, hd, eps)
        oqs[t], okc[pos0 + t] = oracle.rope(oq, ok, H, KV, hd, pos0 + t, base)
        ovc[pos0 + t] = v[t]
    want = oracle.attention_prefill(oqs, okc, ovc, pos0, B, H, KV, hd, scale, sw)
    d = {n: torch.from_numpy(a.copy()).cuda() for n, a in
         dict(q=q, k=k, v=v, kc=kc, vc=vc, norms=norms).items()}
    out = torch.zeros(B, H * hd, device="cuda")
    lib.gncx_hip_attention_prefill(d["q"].data_ptr(), d["k"].data_ptr(), d["v"].data_ptr(), d["kc"].data_ptr(),
                                   d["vc"].data_ptr(), pos0, B, H, KV, hd, scale, sw, d["norms"].data_ptr(), 0,
                                   hd * 4, 1, eps, 0, 0, base, out.data_ptr())
    gncx.check(lib)
    got = out.cpu().numpy().reshape(B, H * hd)
    want = np.asarray(want, np.float32).reshape(B, H * hd)
    errs = [rel_l2(got[t], want[t]) for t in range(B)]
    print(f"prefill device vs oracle pos0={pos0} B={B} sw={sw}: max row rel_l2={max(errs):.2e}")
    assert max(errs) < TOL
    assert rel_l2(d["kc"].cpu().numpy(), okc) < 1e-6
    assert rel_l2(d["vc"].cpu().numpy(), ovc) < 1e-6


@pytest.mark.parametrize("rows,dim", [(5, 4096), (3, 4098), (2, 20000)])
def test_rmsnorm_rows_equals_per_row_calls(lib, rows, dim):
    rng = np.random.default_rng(rows * dim)
    x = (rng.standard_normal((rows, dim)) * 2).astype(np.float32)
    g = synth.make_norm_gamma(dim, 11)
    want = np.zeros_like(x)
    for r in range(rows):
        lib.gncx_rmsnorm_and_encode_4phase(ptr(x[r]), ptr(g), 0, dim, 1e-6, 0, ptr(want[r]), None, None)
    got = np.zeros_like(x)
    lib.gncx_hip_rmsnorm_rows(ptr(x), rows, ptr(g), 0, dim, 1e-6, ptr(got))
    gncx.check(lib)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,dim", [(5, 4096), (3, 4098), (2, 20000), (64, 256)])
def test_add_rmsnorm_rows_equals_add_then_rows(lib, rows, dim):
    """gncx_hip_add_rmsnorm_rows == gncx_hip_vec_add over the rows followed by
    gncx_hip_rmsnorm_rows, bit for bit, in host memory and in place."""
    rng = np.random.default_rng(rows + dim)
    h = (rng.standard_normal((rows, dim)) * 2).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float32)
    g = synth.make_norm_gamma(dim, 12)
    h1, want = h.copy(), np.zeros_like(h)
    lib.gncx_hip_vec_add(ptr(h1), ptr(d), rows * dim)
    lib.gncx_hip_rmsnorm_rows(ptr(h1), rows, ptr(g), 0, dim, 1e-6, ptr(want))
    h2, got = h.copy(), np.zeros_like(h)
    lib.gncx_hip_add_rmsnorm_rows(ptr(h2), ptr(d), rows, ptr(g), 0, dim, 1e-6, ptr(got))
    gncx.check(lib)
    assert np.array_equal(h2, h1) and np.array_equal(got, want)


@pytest.mark.parametrize("n", [1, 7, 4096, 4097, 151936])
def test_argmax_first_of_equal_maxima(lib, n):
    """gncx_hip_argmax: torch.argmax's pick (the first of equal maxima), NaN
    never wins, all -inf gives index 0, and a maximum in the last element of
    a ragged tail is found."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g)
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    cases = [x.clone()]
    if n > 3:
        y = x.clone()
        y[n // 3] = 50.0
        y[n - 1] = 50.0  # equal maximum later: the first one wins
        y[1] = float("nan")
        cases.append(y)
        z = x.clone()
        z[n - 1] = 99.0  # the last element of a ragged tail
        cases.append(z)
    cases.append(torch.full((n,), float("-inf")))
    for c in cases:
        d = c.cuda()
        lib.gncx_hip_argmax(d.data_ptr(), n, out.data_ptr())
        gncx.check(lib)
        want = int(torch.argmax(torch.nan_to_num(c, nan=float("-inf"))).item())
        assert int(out.item()) == want, (n, int(out.item()), want)
