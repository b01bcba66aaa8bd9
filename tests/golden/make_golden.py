"""Write tests/golden/ref_vectors.npz from the reference's own library.

The reference library is oracle/_ref/gncx_llm_core.so, compiled from the
reference's source by oracle/Makefile (the reference ships no tests or
vectors for this path, so these fixtures are the only external pin).  Inputs
are small seeded synthetic tensors; every input and every reference output is
stored, so the fixture stands alone.

Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
import pyoracle  # noqa: E402

sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "gnc-x_amd"))
import synth  # noqa: E402

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
import host_scripts  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "ref_vectors.npz"
TYPES = {"q4_0": 2, "q8_0": 8, "q4_k": 12, "q6_k": 14, "bf16": 30}


def act_probe_weights(k: int) -> np.ndarray:
    """Q8_0 rows that each pick one element with weight 1 (d = 1.0 in fp16),
    so the reference's matvec returns q_m * d_x of its own quantisation."""
    nb = k // 32
    w = np.zeros((k, nb, 34), dtype=np.uint8)
    for m in range(k):
        b, j = divmod(m, 32)
        w[m, b, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
        w[m, b, 2 + j] = 1
    return w.reshape(-1)


def main() -> None:
    ref = pyoracle.Reference()
    rng = np.random.default_rng(20261201)
    data: dict[str, np.ndarray] = {}

    # matvec / matbatch for every type, K = 512 (two super-blocks), N = 48
    k, n, b = 512, 48, 3
    for name, t in TYPES.items():
        w = synth.make_weights(t, n, k, seed=100 + t)
        x = synth.make_activations(1, k, seed=200 + t)
        x[32:64] = 0.0  # one all-zero activation block (the zero-skip paths)
        xb = synth.make_activations(b, k, seed=300 + t)
        data[f"{name}_w"] = w
        data[f"{name}_x"] = x
        data[f"{name}_y"] = ref.matvec(t, w, x, k, n)
        data[f"{name}_xb"] = xb
        data[f"{name}_yb"] = ref.matbatch(t, w, xb, b, k, n)
    data["mv_k"], data["mv_n"], data["mv_b"] = np.int32(k), np.int32(n), np.int32(b)

    # activation quantisation recovered through one-hot Q8_0 rows
    kq = 128
    xq = (rng.standard_normal(kq) * 3).astype(np.float32)
    xq[64:96] = 0.0                              # zero block
    xq[96:128] = np.linspace(-127, 127, 32).astype(np.float32)
    xq[96] = 127.0                               # amax 127 -> inv = 1, exact ties below
    xq[97], xq[98], xq[99], xq[100] = 2.5, 3.5, -2.5, -0.5
    wq = act_probe_weights(kq)
    data["act_x"] = xq
    data["act_probe_y"] = ref.matvec(8, wq, xq, kq, kq)

    # lm_head with softcap (Q6_K tied table)
    vocab, kd = 96, 256
    tab = synth.make_weights(14, vocab, kd, seed=77)
    hx = synth.make_activations(1, kd, seed=78)
    data["lm_w"], data["lm_x"] = tab, hx
    data["lm_y"] = ref.lm_head(14, tab, hx, kd, vocab, 0.0)
    data["lm_y_cap"] = ref.lm_head(14, tab, hx, kd, vocab, 30.0)
    data["lm_vocab"], data["lm_k"] = np.int32(vocab), np.int32(kd)

    # attention: GQA 8/2 x 64, 48 cached rows, step at pos 40 (full + window 16), MQA
    H, KV, hd, rows, pos = 8, 2, 64, 48, 40
    for tag, kv, sw in (("gqa", KV, 0), ("swa", KV, 16), ("mqa", 1, 0)):
        kc = rng.standard_normal((rows, kv * hd)).astype(np.float32)
        vc = rng.standard_normal((rows, kv * hd)).astype(np.float32)
        q = rng.standard_normal(H * hd).astype(np.float32)
        kn = rng.standard_normal(kv * hd).astype(np.float32)
        vn = rng.standard_normal(kv * hd).astype(np.float32)
        out, kc2, vc2 = ref.attention(q, kn, vn, kc, vc, pos, H, kv, hd, 1.0 / np.sqrt(hd), sw, 1)
        assert np.array_equal(kc2[pos], kn) and np.array_equal(vc2[pos], vn)
        for key, val in (("kc", kc), ("vc", vc), ("q", q), ("kn", kn), ("vn", vn), ("out", out)):
            data[f"attn_{tag}_{key}"] = val
        data[f"attn_{tag}_geom"] = np.array([pos, H, kv, hd, sw], dtype=np.int32)

    # per-head RMSNorm, RoPE (with and without factors), RMSNorm, SwiGLU
    v = rng.standard_normal(8 * 128).astype(np.float32)
    gam = synth.make_norm_gamma(128, 5)
    data["rmsh_v"], data["rmsh_g"] = v, gam
    data["rmsh_y"] = ref.rmsnorm_heads(v, gam, 8, 128, 1e-6)
    data["rmsh_y_nog"] = ref.rmsnorm_heads(v, None, 8, 128, 1e-6)
    qv = rng.standard_normal(4 * 128).astype(np.float32)
    kv_ = rng.standard_normal(2 * 128).astype(np.float32)
    fac = (1.0 + rng.random(64)).astype(np.float32)
    data["rope_q"], data["rope_k"], data["rope_f"] = qv, kv_, fac
    for p in (0, 1, 511, 4095, 32767):
        qo, ko = ref.rope(qv, kv_, 4, 2, 128, p, 1e6)
        data[f"rope_q_{p}"], data[f"rope_k_{p}"] = qo, ko
    qo, ko = ref.rope(qv, kv_, 4, 2, 128, 777, 1e4, fac)
    data["rope_q_fac"], data["rope_k_fac"] = qo, ko
    hx = rng.standard_normal(4096).astype(np.float32)
    hg = synth.make_norm_gamma(4096, 6)
    data["rms_x"], data["rms_g"], data["rms_y"] = hx, hg, ref.rmsnorm(hx, hg, 1e-6)
    gx = (rng.standard_normal(2048) * 4).astype(np.float32)
    ux = rng.standard_normal(2048).astype(np.float32)
    data["swi_g"], data["swi_u"], data["swi_y"] = gx, ux, ref.swiglu(gx, ux)

    # the 4-phase encode of the normed vector at several sieve orders
    for lk in (0, 2, 3, 9, 17):
        yk, tk, qk = ref.rmsnorm_encode(hx, hg, 1e-6, lk)
        assert np.array_equal(yk, data["rms_y"])
        data[f"enc_tok_k{lk}"], data[f"enc_qs_k{lk}"] = tk, np.float32(qk)

    # GeGLU over the tanh range and its saturation, with an odd tail
    gg = np.concatenate([np.linspace(-12, 12, 2001), rng.standard_normal(50) * 3]).astype(np.float32)
    gg[7] = 0.0
    ug = rng.standard_normal(gg.size).astype(np.float32)
    data["geg_g"], data["geg_u"], data["geg_y"] = gg, ug, ref.geglu(gg, ug)

    # loader host bookkeeping: layer coordinates and slot-manager call sequences
    data["genome_table"] = host_scripts.genome_table(ref.lib)
    for mf, n_ops, seed in host_scripts.GEO_CASES:
        ops, res = host_scripts.geo_generate(ref.lib, mf, n_ops, 7000 + seed)
        data[f"geo_{mf}_ops"], data[f"geo_{mf}_res"] = ops, res

    # embedding rows (the reference's explicit block decoders)
    for name, t in (("q8_0", 8), ("q6_k", 14), ("bf16", 30)):
        tabe = synth.make_weights(t, 12, 512, seed=500 + t)
        data[f"emb_{name}_tab"] = tabe
        data[f"emb_{name}_y5"] = ref.fetch_embedding(t, tabe, 5, 512, 1.0)
        data[f"emb_{name}_y11s"] = ref.fetch_embedding(t, tabe, 11, 512, 0.37)

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
