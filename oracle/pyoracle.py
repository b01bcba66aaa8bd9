"""ctypes view of the checker libraries (test infrastructure only).

* ``Oracle``     -- libgncx_oracle.so, the C restatement in gncx_oracle.c.
* ``Reference``  -- _ref/gncx_llm_core.so, the reference's own source compiled
                    by oracle/Makefile (present only where it was built).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess
import tempfile

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ORACLE_SO = HERE / "libgncx_oracle.so"
REF_SO = HERE / "_ref" / "gncx_llm_core.so"

_vp, _i32, _f32, _sz = C.c_void_p, C.c_int32, C.c_float, C.c_size_t


def build(quiet: bool = True) -> None:
    """Compile the restatement (and the reference where its source exists)."""
    out = subprocess.run(["make", "-C", str(HERE), "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def _ptr(a) -> int:
    return 0 if a is None else a.ctypes.data


class Oracle:
    """The C restatement.  Methods take/return numpy arrays."""

    def __init__(self, path: os.PathLike | None = None):
        p = pathlib.Path(path) if path else ORACLE_SO
        if not p.exists():
            build()
        lib = C.CDLL(str(p))
        sig = {
            "orc_fp16_to_fp32": (C.c_float, [C.c_uint16]),
            "orc_quantize_act_q8": (None, [_vp, _i32, _vp]),
            "orc_dequant_row": (None, [_i32, _vp, _i32, _vp]),
            "orc_matvec": (None, [_i32, _vp, _vp, _i32, _i32, _vp]),
            "orc_matbatch": (None, [_i32, _vp, _vp, _i32, _i32, _i32, _vp]),
            "orc_lm_head": (None, [_i32, _vp, _vp, _i32, _i32, _f32, _vp]),
            "orc_rmsnorm": (None, [_vp, _vp, _i32, _f32, _vp]),
            "orc_rmsnorm_heads": (None, [_vp, _vp, _i32, _i32, _f32]),
            "orc_rope_table": (None, [_i32, _i32, _f32, _vp, _vp, _vp]),
            "orc_rope": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32]),
            "orc_attention_step": (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
            "orc_attention_prefill": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp]),
            "orc_swiglu": (None, [_vp, _vp, _i32, _vp]),
            "orc_geglu": (None, [_vp, _vp, _i32, _vp]),
            "orc_encode_4phase": (_f32, [_vp, _i32, _i32, _vp]),
            "orc_fetch_embedding": (None, [_i32, _vp, _i32, _i32, _f32, _vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib

    # record layout of orc_act_q8: float d; int32 sum, lo, hi; int8 qs[32]
    ACT_DTYPE = np.dtype([("d", "<f4"), ("sum", "<i4"), ("sum_lo16", "<i4"), ("sum_hi16", "<i4"),
                          ("qs", "i1", (32,))])

    def quantize_act(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.zeros(x.size // 32, dtype=self.ACT_DTYPE)
        self.lib.orc_quantize_act_q8(_ptr(x), x.size, _ptr(out))
        return out

    def dequant(self, ggml_type: int, w: np.ndarray, k: int, n: int, row_bytes: int) -> np.ndarray:
        out = np.empty((n, k), dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        for r in range(n):
            self.lib.orc_dequant_row(ggml_type, w.ctypes.data + r * row_bytes, k, out[r].ctypes.data)
        return out

    def matvec(self, ggml_type: int, w: np.ndarray, x: np.ndarray, k: int, n: int) -> np.ndarray:
        y = np.zeros(n, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.orc_matvec(ggml_type, _ptr(w), _ptr(x), k, n, _ptr(y))
        return y

    def matbatch(self, ggml_type: int, w: np.ndarray, x: np.ndarray, b: int, k: int, n: int) -> np.ndarray:
        y = np.zeros((b, n), dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.orc_matbatch(ggml_type, _ptr(w), _ptr(x), b, k, n, _ptr(y))
        return y

    def lm_head(self, ggml_type, w, x, k, vocab, softcap):
        y = np.zeros(vocab, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.orc_lm_head(ggml_type, _ptr(w), _ptr(x), k, vocab, softcap, _ptr(y))
        return y

    def rmsnorm(self, x, gamma, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self.lib.orc_rmsnorm(_ptr(x), _ptr(np.ascontiguousarray(gamma, dtype=np.float32)), x.size, eps, _ptr(out))
        return out

    def encode(self, v, layer_k):
        """(tokens as packed uint32 words, quant scale) of the 4-phase encode."""
        v = np.ascontiguousarray(v, dtype=np.float32)
        tok = np.zeros(v.size, dtype=np.uint32)
        qs = self.lib.orc_encode_4phase(_ptr(v), v.size, layer_k, _ptr(tok))
        return tok, np.float32(qs)

    def rmsnorm_heads(self, v, gamma, n_heads, head_dim, eps):
        v = np.array(v, dtype=np.float32, copy=True)
        g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
        self.lib.orc_rmsnorm_heads(_ptr(v), _ptr(g), n_heads, head_dim, eps)
        return v

    def rope_table(self, pos, head_dim, base, factors=None):
        c = np.empty(head_dim // 2, dtype=np.float32)
        s = np.empty(head_dim // 2, dtype=np.float32)
        f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
        self.lib.orc_rope_table(pos, head_dim, base, _ptr(f), _ptr(c), _ptr(s))
        return c, s

    def rope(self, q, k, n_heads, n_kv, head_dim, pos, base, factors=None):
        q = None if q is None else np.array(q, dtype=np.float32, copy=True)
        k = None if k is None else np.array(k, dtype=np.float32, copy=True)
        f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
        self.lib.orc_rope(_ptr(q), _ptr(k), _ptr(f), n_heads, n_kv, head_dim, pos, base)
        return q, k

    def attention(self, q, k_new, v_new, k_cache, v_cache, pos, n_heads, n_kv, head_dim, scale, window,
                  write_kv):
        """Returns (out, k_cache, v_cache) with the caches copied, not mutated."""
        kc = np.array(k_cache, dtype=np.float32, copy=True)
        vc = np.array(v_cache, dtype=np.float32, copy=True)
        out = np.zeros(n_heads * head_dim, dtype=np.float32)
        kn = None if k_new is None else np.ascontiguousarray(k_new, dtype=np.float32)
        vn = None if v_new is None else np.ascontiguousarray(v_new, dtype=np.float32)
        self.lib.orc_attention_step(_ptr(np.ascontiguousarray(q, dtype=np.float32)), _ptr(kn), _ptr(vn), _ptr(kc),
                                    _ptr(vc), pos, n_heads, n_kv, head_dim, scale, window, write_kv, _ptr(out))
        return out, kc, vc

    def attention_prefill(self, q, k_cache, v_cache, pos0, b, n_heads, n_kv, head_dim, scale, window):
        """out[b][n_heads*head_dim]: b consecutive attention steps at positions
        pos0 .. pos0+b-1 over caches that already hold those K/V rows."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        kc = np.ascontiguousarray(k_cache, dtype=np.float32)
        vc = np.ascontiguousarray(v_cache, dtype=np.float32)
        assert q.size == b * n_heads * head_dim and kc.shape[0] >= pos0 + b and vc.shape[0] >= pos0 + b
        out = np.zeros((b, n_heads * head_dim), dtype=np.float32)
        self.lib.orc_attention_prefill(_ptr(q), _ptr(kc), _ptr(vc), pos0, b, n_heads, n_kv, head_dim, scale, window,
                                       _ptr(out))
        return out

    def swiglu(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.orc_swiglu(_ptr(g), _ptr(np.ascontiguousarray(u, dtype=np.float32)), g.size, _ptr(out))
        return out

    def geglu(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.orc_geglu(_ptr(g), _ptr(np.ascontiguousarray(u, dtype=np.float32)), g.size, _ptr(out))
        return out

    def fetch_embedding(self, ggml_type, table, token, dim, scale):
        out = np.empty(dim, dtype=np.float32)
        self.lib.orc_fetch_embedding(ggml_type, _ptr(table), token, dim, scale, _ptr(out))
        return out


class Reference:
    """The reference's own library, built from its source by oracle/Makefile.
    Its fp16 table and thread pool are created by gncx_gla_map_readonly
    (cpp:327-330), so construction maps a small temporary file once and never
    unmaps it (unmapping stops the pool, cpp:391-392)."""

    def __init__(self, path: os.PathLike | None = None):
        p = pathlib.Path(path) if path else REF_SO
        if not p.exists():
            raise FileNotFoundError(f"{p} is not built (reference sources absent?)")
        lib = C.CDLL(str(p))
        sig = {
            "gncx_gla_map_readonly": (_vp, [C.c_char_p, _vp]),
            "gncx_xfold_universal_matvec": (None, [_vp, _sz, _i32, _vp, _vp, _i32, _i32, _vp, _vp]),
            "gncx_xfold_universal_matbatch": (None, [_vp, _sz, _i32, _vp, _i32, _i32, _i32, _vp, _vp]),
            "gncx_universal_lm_head_logits": (None, [_vp, _sz, _i32, _vp, _i32, _i32, _f32, _vp]),
            "gncx_mqa_attention_step_ext": (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32,
                                                   _i32, _vp]),
            "gncx_rmsnorm_inplace_heads": (None, [_vp, _vp, _sz, _i32, _i32, _i32, _f32]),
            "gncx_apply_rope_xor11_ext": (None, [_vp, _vp, _vp, _vp, _sz, _i32, _i32, _i32, _i32, _i32, _f32]),
            "gncx_rmsnorm_and_encode_4phase": (None, [_vp, _vp, _sz, _i32, _f32, _i32, _vp, _vp, _vp]),
            "gncx_swiglu_activation": (None, [_vp, _vp, _i32, _vp]),
            "gncx_geglu_activation": (None, [_vp, _vp, _i32, _vp]),
            "gncx_genome_get_layer_coordinate": (None, [_i32, _i32, _i32, _vp, _vp, _vp, _vp]),
            "gncx_geo_mm_create": (_vp, [C.c_uint32]),
            "gncx_geo_mm_destroy": (None, [_vp]),
            "gncx_geo_alloc": (_i32, [_vp, C.c_uint8, _vp, _vp, _vp, _vp]),
            "gncx_geo_free": (None, [_vp, C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint32]),
            "gncx_geo_fragmentation": (_f32, [_vp]),
            "gncx_geo_used": (_sz, [_vp]),
            "gncx_geo_capacity": (_sz, [_vp]),
            "gncx_fetch_token_embedding_q8_0": (None, [_vp, _sz, _i32, _i32, _f32, _vp]),
            "gncx_fetch_token_embedding_q6_k": (None, [_vp, _sz, _i32, _i32, _f32, _vp]),
            "gncx_fetch_token_embedding_bf16": (None, [_vp, _sz, _i32, _i32, _f32, _vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        fd, tmp = tempfile.mkstemp(prefix="gncx_ref_map_")
        os.write(fd, b"\0" * 64)
        os.close(fd)
        self._handle = lib.gncx_gla_map_readonly(tmp.encode(), None)
        os.unlink(tmp)
        self.lib = lib

    def matvec(self, ggml_type, w, x, k, n):
        y = np.zeros(n, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.gncx_xfold_universal_matvec(_ptr(w), 0, ggml_type, _ptr(x), None, k, n, _ptr(y), None)
        return y

    def matbatch(self, ggml_type, w, x, b, k, n):
        y = np.zeros((b, n), dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.gncx_xfold_universal_matbatch(_ptr(w), 0, ggml_type, _ptr(x), b, k, n, _ptr(y), None)
        return y

    def lm_head(self, ggml_type, w, x, k, vocab, softcap):
        y = np.zeros(vocab, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib.gncx_universal_lm_head_logits(_ptr(w), 0, ggml_type, _ptr(x), k, vocab, softcap, _ptr(y))
        return y

    def attention(self, q, k_new, v_new, k_cache, v_cache, pos, n_heads, n_kv, head_dim, scale, window,
                  write_kv):
        kc = np.array(k_cache, dtype=np.float32, copy=True)
        vc = np.array(v_cache, dtype=np.float32, copy=True)
        out = np.zeros(n_heads * head_dim, dtype=np.float32)
        kn = None if k_new is None else np.ascontiguousarray(k_new, dtype=np.float32)
        vn = None if v_new is None else np.ascontiguousarray(v_new, dtype=np.float32)
        self.lib.gncx_mqa_attention_step_ext(_ptr(np.ascontiguousarray(q, dtype=np.float32)), _ptr(kn), _ptr(vn),
                                             _ptr(kc), _ptr(vc), pos, n_heads, n_kv, head_dim, scale, window,
                                             write_kv, _ptr(out))
        return out, kc, vc

    def rmsnorm_heads(self, v, gamma, n_heads, head_dim, eps):
        v = np.array(v, dtype=np.float32, copy=True)
        if gamma is None:
            self.lib.gncx_rmsnorm_inplace_heads(_ptr(v), None, 0, 0, n_heads, head_dim, eps)
        else:
            g = np.ascontiguousarray(gamma, dtype=np.float32)
            self.lib.gncx_rmsnorm_inplace_heads(_ptr(v), _ptr(g), 0, 1, n_heads, head_dim, eps)
        return v

    def rope(self, q, k, n_heads, n_kv, head_dim, pos, base, factors=None):
        q = None if q is None else np.array(q, dtype=np.float32, copy=True)
        k = None if k is None else np.array(k, dtype=np.float32, copy=True)
        if factors is None:
            self.lib.gncx_apply_rope_xor11_ext(_ptr(q), _ptr(k), None, None, 0, 0, n_heads, n_kv, head_dim, pos,
                                               base)
        else:
            f = np.ascontiguousarray(factors, dtype=np.float32)
            self.lib.gncx_apply_rope_xor11_ext(_ptr(q), _ptr(k), None, _ptr(f), 0, 1, n_heads, n_kv, head_dim, pos,
                                               base)
        return q, k

    def rmsnorm(self, x, gamma, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        g = np.ascontiguousarray(gamma, dtype=np.float32)
        self.lib.gncx_rmsnorm_and_encode_4phase(_ptr(x), _ptr(g), 0, x.size, eps, 0, _ptr(out), None, None)
        return out

    def rmsnorm_encode(self, x, gamma, eps, layer_k):
        """(normed, tokens as packed uint32 words, quant scale)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        tok = np.zeros(x.size, dtype=np.uint32)
        qs = np.zeros(1, dtype=np.float32)
        g = np.ascontiguousarray(gamma, dtype=np.float32)
        self.lib.gncx_rmsnorm_and_encode_4phase(_ptr(x), _ptr(g), 0, x.size, eps, layer_k, _ptr(out), _ptr(tok),
                                                _ptr(qs))
        return out, tok, qs[0]

    def swiglu(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.gncx_swiglu_activation(_ptr(g), _ptr(np.ascontiguousarray(u, dtype=np.float32)), g.size, _ptr(out))
        return out

    def geglu(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.gncx_geglu_activation(_ptr(g), _ptr(np.ascontiguousarray(u, dtype=np.float32)), g.size, _ptr(out))
        return out

    def fetch_embedding(self, ggml_type, table, token, dim, scale):
        out = np.empty(dim, dtype=np.float32)
        fn = {8: self.lib.gncx_fetch_token_embedding_q8_0, 14: self.lib.gncx_fetch_token_embedding_q6_k,
              30: self.lib.gncx_fetch_token_embedding_bf16}[ggml_type]
        fn(_ptr(table), 0, token, dim, scale, _ptr(out))
        return out
