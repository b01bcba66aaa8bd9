"""Pins the oracle (CPU).  Each check is chosen so that a plausible mistake in
the restatement -- a wrong nibble/bit index, a dropped term, a wrong rounding
mode, a transposed operand -- fails it: IEEE tables, closed forms, packers
written in the opposite (quantising) direction, float64 brute force, and the
reference's own outputs (tests/golden/ref_vectors.npz, from
tests/golden/make_golden.py)."""
from __future__ import annotations

import numpy as np
import pytest

import synth
from conftest import gncx, rel_l2

Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 2, 8, 12, 14, 30
F16_ONE = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)


def f16_bytes(v: float) -> np.ndarray:
    return np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)


# ---------------------------------------------------------------- decoders

def test_fp16_decode_all_codes(oracle):
    """cpp:85-112 is an exact IEEE half->float: compare all 65536 bit patterns
    with numpy's conversion (NaNs only as NaNs: the value crosses ctypes as a
    double, which may quiet a signalling NaN)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = codes.view(np.float16).astype(np.float32).view(np.uint32)
    f = oracle.lib.orc_fp16_to_fp32
    got = np.array([np.float32(f(int(c))).view(np.uint32) for c in codes], dtype=np.uint32)
    finite = ~np.isnan(codes.view(np.float16))
    assert np.array_equal(got[finite], want[finite])
    assert np.all(np.isnan(got[~finite].view(np.float32)))


def pack_q4_0(d: float, q: np.ndarray) -> np.ndarray:
    """ggml Q4_0 packing: qs[j] = q[j] | q[j+16] << 4, q in [0, 15]."""
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = f16_bytes(d)
    blk[2:18] = (q[:16] | (q[16:] << 4)).astype(np.uint8)
    return blk


def pack_q4_k(d: float, dmin: float, sc: np.ndarray, mn: np.ndarray, q: np.ndarray) -> np.ndarray:
    """ggml Q4_K packing (quantising direction): 6-bit scales/mins of the 8
    sub-blocks into 12 bytes; nibble chunk c holds elements 64c+l (low) and
    64c+32+l (high)."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16_bytes(d), f16_bytes(dmin)
    s = np.zeros(12, dtype=np.uint8)
    for j in range(8):
        if j < 4:
            s[j] = sc[j] & 63
            s[j + 4] = mn[j] & 63
        else:
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    blk[4:16] = s
    for c in range(4):
        lo = q[64 * c:64 * c + 32]
        hi = q[64 * c + 32:64 * c + 64]
        blk[16 + 32 * c:48 + 32 * c] = (lo | (hi << 4)).astype(np.uint8)
    return blk


def pack_q6_k(d: float, sc: np.ndarray, q: np.ndarray) -> np.ndarray:
    """ggml Q6_K packing: per 128-half, ql[l] = q1|q3<<4, ql[l+32] = q2|q4<<4,
    qh[l] = hi2(q1) | hi2(q2)<<2 | hi2(q3)<<4 | hi2(q4)<<6 with q1..q4 the
    elements l, l+32, l+64, l+96 (stored q = value + 32 in [0, 63])."""
    blk = np.zeros(210, dtype=np.uint8)
    for h in range(2):
        qq = q[128 * h:128 * h + 128]
        for l in range(32):
            q1, q2, q3, q4 = int(qq[l]), int(qq[l + 32]), int(qq[l + 64]), int(qq[l + 96])
            blk[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            blk[64 * h + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            blk[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blk[192:208] = sc.astype(np.int8).view(np.uint8)
    blk[208:210] = f16_bytes(d)
    return blk


def test_dequant_q4_0_packer(oracle):
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, 32).astype(np.uint8)
    blk = pack_q4_0(0.75, q)
    got = oracle.dequant(Q4_0, blk, 32, 1, 18)[0]
    assert np.array_equal(got, np.float32(0.75) * (q.astype(np.float32) - 8))


def test_dequant_q8_0_closed_form(oracle):
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = f16_bytes(0.5)
    vals = np.arange(-16, 16, dtype=np.int8)
    blk[2:] = vals.view(np.uint8)
    assert np.array_equal(oracle.dequant(Q8_0, blk, 32, 1, 34)[0], vals.astype(np.float32) * 0.5)


def test_dequant_q4_k_packer(oracle):
    rng = np.random.default_rng(2)
    for _ in range(20):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        d, dmin = float(np.float16(rng.random() * 0.05)), float(np.float16(rng.random() * 0.05))
        blk = pack_q4_k(d, dmin, sc, mn, q)
        got = oracle.dequant(Q4_K, blk, 256, 1, 144)[0]
        sub = np.arange(256) // 32
        # every product is exact in float64 and float32 here, the difference rounds once
        want = (np.float64(d) * sc[sub] * q - np.float64(dmin) * mn[sub]).astype(np.float32)
        assert np.array_equal(got, want)


def test_dequant_q6_k_packer(oracle):
    rng = np.random.default_rng(3)
    for _ in range(20):
        sc = rng.integers(-32, 32, 16)
        q = rng.integers(0, 64, 256)
        d = float(np.float16(rng.random() * 0.05))
        blk = pack_q6_k(d, sc, q)
        got = oracle.dequant(Q6_K, blk, 256, 1, 210)[0]
        e = np.arange(256)
        sidx = (e // 128) * 8 + (e % 32) // 16 + 2 * ((e % 128) // 32)
        want = (np.float32(d) * sc[sidx].astype(np.float32)) * (q - 32).astype(np.float32)
        assert np.array_equal(got, want.astype(np.float32))


def test_embedding_decoders_match_reference(oracle, golden):
    """The reference's explicit decoders (cpp:693-780), bit for bit."""
    for name, t in (("q8_0", Q8_0), ("q6_k", Q6_K), ("bf16", BF16)):
        tab = golden[f"emb_{name}_tab"]
        assert np.array_equal(oracle.fetch_embedding(t, tab, 5, 512, 1.0), golden[f"emb_{name}_y5"])
        assert np.array_equal(oracle.fetch_embedding(t, tab, 11, 512, 0.37), golden[f"emb_{name}_y11s"])


# ------------------------------------------------------- activation quant

def test_act_quant_known_answers(oracle):
    x = np.zeros(96, dtype=np.float32)
    x[0:32] = np.linspace(-1, 1, 32)            # amax 1 at both ends
    x[32] = 127.0                               # amax 127: inv = 1, d = 1
    x[33:37] = [2.5, 3.5, -2.5, -0.5]           # ties to even
    a = oracle.quantize_act(x)
    assert a["qs"][0][0] == -127 and a["qs"][0][31] == 127
    assert a["d"][0] == np.float32(1.0) / np.float32(127.0)
    assert a["d"][1] == 1.0
    assert list(a["qs"][1][1:5]) == [2, 4, -2, 0]
    assert a["d"][2] == 0 and not a["qs"][2].any() and a["sum"][2] == 0
    assert np.all(np.abs(a["qs"].astype(int)) <= 127)
    assert np.array_equal(a["sum_lo16"], a["qs"][:, :16].astype(int).sum(1))
    assert np.array_equal(a["sum_hi16"], a["qs"][:, 16:].astype(int).sum(1))
    assert np.array_equal(a["sum"], a["sum_lo16"] + a["sum_hi16"])


def test_act_quant_matches_reference_probe(oracle, golden):
    """The reference's Q8_0 matvec over one-hot rows returns q_m * d_x of its
    own quantisation: recover q_m and compare (cpp:955-995)."""
    x = golden["act_x"]
    y = golden["act_probe_y"]
    a = oracle.quantize_act(x)
    d = np.repeat(a["d"], 32)
    qs = a["qs"].reshape(-1).astype(np.float64)
    nz = d > 0
    q_ref = np.zeros_like(qs)
    q_ref[nz] = np.rint(y[nz].astype(np.float64) / d[nz])
    assert np.array_equal(q_ref[nz], qs[nz])
    assert np.all(y[~nz] == 0)
    # d is the IEEE quotient amax / 127
    amax = np.abs(x.reshape(-1, 32)).max(1).astype(np.float32)
    assert np.array_equal(a["d"], np.where(amax > 0, amax / np.float32(127), 0).astype(np.float32))


# ---------------------------------------------------- dots and matvec

TYPES = [Q4_0, Q8_0, Q4_K, Q6_K, BF16]


@pytest.mark.parametrize("t", TYPES)
def test_matvec_vs_float64_bruteforce(oracle, t):
    """y = dequant(W) . dequant(Q8(x)) in float64 (BF16: fp32 x)."""
    k, n = 1024, 40
    w = synth.make_weights(t, n, k, seed=11 + t)
    x = synth.make_activations(1, k, seed=12 + t)
    W = oracle.dequant(t, w, k, n, gncx.row_bytes(t, k)).astype(np.float64)
    if t == BF16:
        xv = x.astype(np.float64)
    else:
        a = oracle.quantize_act(x)
        xv = (a["qs"].astype(np.float64) * a["d"][:, None].astype(np.float64)).reshape(-1)
    assert rel_l2(oracle.matvec(t, w, x, k, n), W @ xv) < 2e-6


@pytest.mark.parametrize("name,t", [("q4_0", Q4_0), ("q8_0", Q8_0), ("q4_k", Q4_K), ("q6_k", Q6_K), ("bf16", BF16)])
def test_matvec_matbatch_match_reference(oracle, golden, name, t):
    k, n, b = int(golden["mv_k"]), int(golden["mv_n"]), int(golden["mv_b"])
    w = golden[f"{name}_w"]
    assert rel_l2(oracle.matvec(t, w, golden[f"{name}_x"], k, n), golden[f"{name}_y"]) < 1e-6
    assert rel_l2(oracle.matbatch(t, w, golden[f"{name}_xb"], b, k, n), golden[f"{name}_yb"]) < 1e-6


def test_special_cases(oracle):
    k, n = 256, 8
    # Q8_0, d_w = 1 and activations with amax 127 in every block (d_x = 1): a plain int dot
    rng = np.random.default_rng(4)
    w = synth.make_weights(Q8_0, n, k, seed=5).reshape(n, k // 32, 34)
    w[:, :, 0:2] = F16_ONE
    x = rng.integers(-126, 127, k).astype(np.float32)
    x[::32] = 127.0
    wi = w[:, :, 2:].reshape(n, k).view(np.int8).astype(np.int64)
    assert np.array_equal(oracle.matvec(Q8_0, w.reshape(-1), x, k, n), (wi @ x.astype(np.int64)).astype(np.float32))
    # Q4_0 with every nibble = 8 is zero
    w4 = synth.make_weights(Q4_0, n, k, seed=6).reshape(n, k // 32, 18)
    w4[:, :, 2:] = 0x88
    assert not oracle.matvec(Q4_0, w4.reshape(-1), synth.make_activations(1, k, 7), k, n).any()
    # Q6_K with every stored q = 32 (ql = 0, qh bits = 0b10) is zero
    w6 = synth.make_weights(Q6_K, n, k, seed=8).reshape(n, 1, 210)
    w6[:, :, 0:128] = 0
    w6[:, :, 128:192] = 0xAA
    assert not oracle.matvec(Q6_K, w6.reshape(-1), synth.make_activations(1, k, 9), k, n).any()
    # Q4_K with dmin = 0 is a scaled int4 dot: d*sc*q against the Q8 activations
    w4k = synth.make_weights(Q4_K, n, k, seed=10).reshape(n, 144)
    w4k[:, 2:4] = 0
    xk = synth.make_activations(1, k, 11)
    W = oracle.dequant(Q4_K, w4k.reshape(-1), k, n, 144).astype(np.float64)
    assert np.all(W[W != 0] > 0)  # no offset term left
    a = oracle.quantize_act(xk)
    xv = (a["qs"].astype(np.float64) * a["d"][:, None]).reshape(-1)
    assert rel_l2(oracle.matvec(Q4_K, w4k.reshape(-1), xk, k, n), W @ xv) < 2e-6


def test_matbatch_rows_are_matvecs(oracle):
    k, n, b = 512, 16, 5
    for t in TYPES:
        w = synth.make_weights(t, n, k, seed=20 + t)
        X = synth.make_activations(b, k, seed=21 + t)
        Y = oracle.matbatch(t, w, X, b, k, n)
        for r in range(b):
            assert rel_l2(Y[r], oracle.matvec(t, w, X[r], k, n)) < 1e-6


def test_lm_head_matches_reference(oracle, golden):
    w, x = golden["lm_w"], golden["lm_x"]
    v, k = int(golden["lm_vocab"]), int(golden["lm_k"])
    assert rel_l2(oracle.lm_head(Q6_K, w, x, k, v, 0.0), golden["lm_y"]) < 1e-6
    capped = oracle.lm_head(Q6_K, w, x, k, v, 30.0)
    assert rel_l2(capped, golden["lm_y_cap"]) < 1e-6
    assert np.all(np.abs(capped) <= 30.0)


# ------------------------------------------------ norms, rope, attention

def test_rmsnorm_heads_closed_forms(oracle, golden):
    v = np.full(4 * 64, 2.0, dtype=np.float32)
    out = oracle.rmsnorm_heads(v, None, 4, 64, 1e-6)
    assert np.allclose(out, 2.0 / np.sqrt(4.0 + 1e-6), rtol=2e-7, atol=0)
    rng = np.random.default_rng(6)
    u = rng.standard_normal(4 * 64).astype(np.float32)
    assert np.array_equal(oracle.rmsnorm_heads(u, None, 4, 64, 0.0), oracle.rmsnorm_heads(2 * u, None, 4, 64, 0.0))
    # the reference build contracts the square-sum into FMAs: last-bit differences only
    assert rel_l2(oracle.rmsnorm_heads(golden["rmsh_v"], golden["rmsh_g"], 8, 128, 1e-6), golden["rmsh_y"]) < 1e-6
    assert rel_l2(oracle.rmsnorm_heads(golden["rmsh_v"], None, 8, 128, 1e-6), golden["rmsh_y_nog"]) < 1e-6


def test_rmsnorm_matches_reference(oracle, golden):
    assert rel_l2(oracle.rmsnorm(golden["rms_x"], golden["rms_g"], 1e-6), golden["rms_y"]) < 1e-6


def test_rope_closed_forms(oracle, golden):
    q, k = golden["rope_q"], golden["rope_k"]
    q0, k0 = oracle.rope(q, k, 4, 2, 128, 0, 1e6)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    c, s = oracle.rope_table(32767, 128, 1e6)
    theta = 32767.0 / (1e6 ** (np.arange(64) * 2.0 / 128))
    assert np.allclose(c, np.cos(theta), atol=2e-3) and np.allclose(s, np.sin(theta), atol=2e-3)
    for p in (1, 511, 4095, 32767):
        qp, kp = oracle.rope(q, k, 4, 2, 128, p, 1e6)
        # per-pair norms are preserved
        qa, qb = q.reshape(4, 2, 64), qp.reshape(4, 2, 64)
        assert np.allclose(np.hypot(qa[:, 0], qa[:, 1]), np.hypot(qb[:, 0], qb[:, 1]), rtol=1e-5)
        assert rel_l2(qp, golden[f"rope_q_{p}"]) < 1e-6 and rel_l2(kp, golden[f"rope_k_{p}"]) < 1e-6
    qf, kf = oracle.rope(q, k, 4, 2, 128, 777, 1e4, golden["rope_f"])
    assert rel_l2(qf, golden["rope_q_fac"]) < 1e-6 and rel_l2(kf, golden["rope_k_fac"]) < 1e-6


def attn_case(rng, H, KV, hd, rows):
    kc = rng.standard_normal((rows, KV * hd)).astype(np.float32)
    vc = rng.standard_normal((rows, KV * hd)).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kn = rng.standard_normal(KV * hd).astype(np.float32)
    vn = rng.standard_normal(KV * hd).astype(np.float32)
    return q, kn, vn, kc, vc


def test_attention_closed_forms(oracle):
    rng = np.random.default_rng(7)
    H, KV, hd, rows = 8, 2, 64, 40
    q, kn, vn, kc, vc = attn_case(rng, H, KV, hd, rows)
    sc = 1 / np.sqrt(hd)
    # pos 0: softmax over one row is exactly 1 -> out = v_new per head
    out, kc2, vc2 = oracle.attention(q, kn, vn, kc, vc, 0, H, KV, hd, sc, 0, 1)
    assert np.array_equal(out.reshape(H, hd), np.repeat(vn.reshape(KV, hd), H // KV, axis=0))
    assert np.array_equal(kc2[0], kn) and np.array_equal(vc2[0], vn)
    # window 1 at pos 30 -> out = v_new
    out, _, _ = oracle.attention(q, kn, vn, kc, vc, 30, H, KV, hd, sc, 1, 1)
    assert np.array_equal(out.reshape(H, hd), np.repeat(vn.reshape(KV, hd), H // KV, axis=0))
    # identical keys -> mean of the V window
    kc_eq = np.tile(kn, (rows, 1))
    out, _, vcw = oracle.attention(q, kn, vn, kc_eq, vc, 25, H, KV, hd, sc, 0, 1)
    mean_v = vcw[:26].reshape(26, KV, hd).mean(0)
    assert np.allclose(out.reshape(H, hd), np.repeat(mean_v, H // KV, axis=0), rtol=0, atol=2e-6)
    # write_kv = 0: the cache row at pos is used as stored
    out0, kc0, _ = oracle.attention(q, kn, vn, kc, vc, 20, H, KV, hd, sc, 0, 0)
    assert np.array_equal(kc0, kc)


def test_attention_mqa_is_replicated_gqa(oracle):
    rng = np.random.default_rng(8)
    H, hd, rows = 8, 64, 30
    q, kn, vn, kc, vc = attn_case(rng, H, 1, hd, rows)
    o1, _, _ = oracle.attention(q, kn, vn, kc, vc, 22, H, 1, hd, 0.125, 0, 1)
    o2, _, _ = oracle.attention(q, np.tile(kn, H), np.tile(vn, H), np.tile(kc, (1, H)), np.tile(vc, (1, H)), 22,
                                H, H, hd, 0.125, 0, 1)
    assert np.array_equal(o1, o2)


def test_attention_window_is_a_shorter_cache(oracle):
    rng = np.random.default_rng(9)
    H, KV, hd, rows, pos, W = 4, 2, 64, 50, 45, 12
    q, kn, vn, kc, vc = attn_case(rng, H, KV, hd, rows)
    o1, _, _ = oracle.attention(q, kn, vn, kc, vc, pos, H, KV, hd, 0.125, W, 1)
    o2, _, _ = oracle.attention(q, kn, vn, kc[pos - W + 1:pos + 1], vc[pos - W + 1:pos + 1], W - 1, H, KV, hd,
                                0.125, 0, 1)
    assert np.array_equal(o1, o2)


@pytest.mark.parametrize("H,KV,W,pos0", [(8, 2, 0, 0), (8, 2, 7, 0), (8, 1, 0, 5), (4, 4, 16, 3)])
def test_attention_prefill_is_consecutive_steps(oracle, H, KV, W, pos0):
    """The batched causal pass (the streamer's prefill loop, lua/gncx_streamer.lua
    1079-1109) equals b consecutive single steps that each write their K/V row,
    bit for bit: GQA, a sliding window shorter than the batch, MQA after a
    cached prefix, and one KV head per query head."""
    rng = np.random.default_rng(31 + H + KV + W)
    hd, b = 64, 37
    rows = pos0 + b
    kc = np.zeros((rows, KV * hd), np.float32)
    vc = np.zeros((rows, KV * hd), np.float32)
    kc[:pos0] = rng.standard_normal((pos0, KV * hd), dtype=np.float32)
    vc[:pos0] = rng.standard_normal((pos0, KV * hd), dtype=np.float32)
    q = rng.standard_normal((b, H * hd), dtype=np.float32)
    kn = rng.standard_normal((b, KV * hd), dtype=np.float32)
    vn = rng.standard_normal((b, KV * hd), dtype=np.float32)
    sc = 1 / np.sqrt(hd)
    want = np.zeros((b, H * hd), np.float32)
    kcs, vcs = kc.copy(), vc.copy()
    for i in range(b):
        want[i], kcs, vcs = oracle.attention(q[i], kn[i], vn[i], kcs, vcs, pos0 + i, H, KV, hd, sc, W, 1)
    got = oracle.attention_prefill(q, kcs, vcs, pos0, b, H, KV, hd, sc, W)
    assert np.array_equal(got, want)


def test_attention_prefill_matches_reference_steps(oracle, ref):
    """Against the reference's own step, called once per position."""
    rng = np.random.default_rng(44)
    H, KV, hd, b = 8, 2, 128, 40
    kc = np.zeros((b, KV * hd), np.float32)
    vc = np.zeros((b, KV * hd), np.float32)
    q = rng.standard_normal((b, H * hd), dtype=np.float32)
    kn = rng.standard_normal((b, KV * hd), dtype=np.float32)
    vn = rng.standard_normal((b, KV * hd), dtype=np.float32)
    want = np.zeros((b, H * hd), np.float32)
    for i in range(b):
        want[i], kc, vc = ref.attention(q[i], kn[i], vn[i], kc, vc, i, H, KV, hd, 1 / np.sqrt(hd), 0, 1)
    got = oracle.attention_prefill(q, kc, vc, 0, b, H, KV, hd, 1 / np.sqrt(hd), 0)
    assert rel_l2(got, want) < 1e-6


@pytest.mark.parametrize("tag", ["gqa", "swa", "mqa"])
def test_attention_matches_reference(oracle, golden, tag):
    g = golden
    pos, H, kv, hd, sw = (int(v) for v in g[f"attn_{tag}_geom"])
    out, kc, vc = oracle.attention(g[f"attn_{tag}_q"], g[f"attn_{tag}_kn"], g[f"attn_{tag}_vn"], g[f"attn_{tag}_kc"],
                                   g[f"attn_{tag}_vc"], pos, H, kv, hd, 1.0 / np.sqrt(hd), sw, 1)
    assert rel_l2(out, g[f"attn_{tag}_out"]) < 1e-6


def test_swiglu(oracle, golden):
    assert np.array_equal(oracle.swiglu(golden["swi_g"], golden["swi_u"]), golden["swi_y"])
    z = oracle.swiglu(np.array([0.0, -100.0], np.float32), np.array([3.0, 3.0], np.float32))
    assert z[0] == 0.0 and abs(z[1]) < 1e-30


def test_geglu(oracle, golden):
    """The reference library may contract x + 0.044715 x^3 into an FMA; the
    oracle does not, so the bar is 1e-6 relative L2 plus the closed forms:
    GELU(0) = 0, x * u where tanh saturates to 1, 0 where it saturates to -1."""
    g, u = golden["geg_g"], golden["geg_u"]
    y = oracle.geglu(g, u)
    assert rel_l2(y, golden["geg_y"]) < 1e-6
    assert y[7] == 0.0
    hi, lo = g >= 10.0, g <= -10.0
    assert np.array_equal(y[hi], (0.5 * g[hi] * 2.0 * u[hi]).astype(np.float32))
    assert np.all(np.abs(y[lo]) < 1e-6)
    # float64 evaluation of the same formula
    x = g.astype(np.float64)
    want = 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3))) * u
    assert rel_l2(y, want) < 1e-6


@pytest.mark.parametrize("lk", [0, 2, 3, 9, 17])
def test_encode_4phase(oracle, golden, lk):
    """Tokens and quant scale bit-exact with the reference's encode of the
    same normed vector; the tokens reconstruct the rounded integers
    sign * d R_k + residual (|residual| below 2^16 here) and, at k = 0
    (R_k = 1), d is the integer itself with no residual."""
    v = golden["rms_y"]
    tok, qs = oracle.encode(v, lk)
    assert np.array_equal(tok, golden[f"enc_tok_k{lk}"])
    assert qs == golden[f"enc_qs_k{lk}"]
    phase, d, ares = tok & 0xFF, (tok >> 8) & 0xFF, (tok >> 16).astype(np.int64)
    r_k = int("1" * (lk + 1))
    sign = np.where(phase >> 1, 1, -1)
    rsign = np.where(phase & 1, 1, -1)
    val = sign * d.astype(np.int64) * r_k + rsign * ares
    target = np.float32(9 * r_k)
    to_int = target / np.float32(np.abs(v).max())
    want = np.rint((v * to_int).astype(np.float32)).astype(np.int64)
    if lk <= 3:
        assert np.array_equal(val, want)
    if lk == 0:
        assert np.array_equal(d.astype(np.int64), np.abs(want)) and np.all(ares == 0)
    assert np.all(d <= 9)


def test_oracle_against_live_reference(oracle, ref):
    """Where the reference library is built (this container), compare on a
    fresh seed as well."""
    k, n = 2048, 24
    for t in TYPES:
        w = synth.make_weights(t, n, k, seed=900 + t)
        x = synth.make_activations(1, k, seed=901 + t)
        assert rel_l2(oracle.matvec(t, w, x, k, n), ref.matvec(t, w, x, k, n)) < 1e-6


def test_oracle_model_prefill_equals_token_steps(oracle):
    """The oracle's batched prefill (matbatch projections, the batched causal
    attention pass) against the same model stepped token by token (matvec
    projections, one attention step each): logits after the prompt and after
    a decode step that reads the prefilled caches agree to matbatch-versus-
    matvec summation order."""
    import torch

    import gncx_amd.decode as dec
    from oracle_model import OracleModel

    shape = dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=512, vocab=600)
    model = dec.build_model(torch, shape, seed=17, device="cpu")
    prompt = [5, 17, 599, 0, 311, 42, 7, 128, 64, 1]
    a, b = OracleModel(oracle, model, max_seq=16), OracleModel(oracle, model, max_seq=16)
    for pos, tok in enumerate(prompt[:-1]):
        a.step(tok, pos, logits=False)
    want = a.step(prompt[-1], len(prompt) - 1)
    got = b.prefill(prompt)
    assert rel_l2(got, want) < 1e-5
    for l in range(shape.n_layers):  # every layer's K/V rows, the last layer's included
        assert rel_l2(b.kc[l][:len(prompt)], a.kc[l][:len(prompt)]) < 1e-5
        assert rel_l2(b.vc[l][:len(prompt)], a.vc[l][:len(prompt)]) < 1e-5
    tok = int(np.argmax(want))
    assert rel_l2(b.step(tok, len(prompt)), a.step(tok, len(prompt))) < 1e-5
