"""The Qwen3 branch of GNCXStreamer:forward_token (lua/gncx_streamer.lua:759-965)
composed from oracle functions on the CPU: RMSNorm, Q/K/V matvecs, per-head
Q/K RMSNorm, NEOX RoPE, attention with a KV write at pos, output projection
and residual, RMSNorm, gate/up, SwiGLU, down and residual, then the final
norm and the tied lm_head.  Test infrastructure: the reference the decode
tests compare the library's logits with."""
from __future__ import annotations

import numpy as np

from conftest import gncx


class OracleModel:
    """The streamer's Qwen3 step from oracle pieces over a host copy of the blob."""

    def __init__(self, oracle, model, max_seq: int = 64):
        self.o, self.s = oracle, model.shape
        self.blob = model.blob.cpu().numpy() if hasattr(model.blob, "cpu") else np.asarray(model.blob)
        self.off = model.offsets
        s = self.s
        self.kc = [np.zeros((max_seq, s.kv_dim), np.float32) for _ in range(s.n_layers)]
        self.vc = [np.zeros((max_seq, s.kv_dim), np.float32) for _ in range(s.n_layers)]

    def w(self, name, rows, cols, t):
        o = self.off[name]
        return self.blob[o:o + gncx.row_bytes(t, cols) * rows]

    def f(self, name, n):
        o = self.off[name]
        return self.blob[o:o + 4 * n].view(np.float32)

    def step(self, token, pos, logits: bool = True):
        """Logits after token at pos (None with logits=False: the KV caches
        advance, as for the streamer's prompt tokens before the last)."""
        o, s = self.o, self.s
        E, lt = s.embed, s.layer_type
        table = self.w("token_embd.weight", s.vocab, E, s.embd_type)
        h = o.fetch_embedding(s.embd_type, table, token, E, 1.0)
        for l in range(s.n_layers):
            p = f"blk.{l}"
            x = o.rmsnorm(h, self.f(f"{p}.attn_norm.weight", E), s.eps)
            q = o.matvec(lt, self.w(f"{p}.attn_q.weight", s.q_dim, E, lt), x, E, s.q_dim)
            k = o.matvec(lt, self.w(f"{p}.attn_k.weight", s.kv_dim, E, lt), x, E, s.kv_dim)
            v = o.matvec(lt, self.w(f"{p}.attn_v.weight", s.kv_dim, E, lt), x, E, s.kv_dim)
            q = o.rmsnorm_heads(q, self.f(f"{p}.attn_q_norm.weight", s.head_dim), s.n_heads, s.head_dim, s.eps)
            k = o.rmsnorm_heads(k, self.f(f"{p}.attn_k_norm.weight", s.head_dim), s.n_kv, s.head_dim, s.eps)
            q, k = o.rope(q, k, s.n_heads, s.n_kv, s.head_dim, pos, s.rope_base)
            a, self.kc[l], self.vc[l] = o.attention(q, k, v, self.kc[l], self.vc[l], pos, s.n_heads, s.n_kv,
                                                    s.head_dim, 1.0 / np.sqrt(s.head_dim), 0, 1)
            h = h + o.matvec(lt, self.w(f"{p}.attn_output.weight", E, s.q_dim, lt), a, s.q_dim, E)
            x = o.rmsnorm(h, self.f(f"{p}.ffn_norm.weight", E), s.eps)
            g = o.matvec(lt, self.w(f"{p}.ffn_gate.weight", s.ffn, E, lt), x, E, s.ffn)
            u = o.matvec(lt, self.w(f"{p}.ffn_up.weight", s.ffn, E, lt), x, E, s.ffn)
            h = h + o.matvec(lt, self.w(f"{p}.ffn_down.weight", E, s.ffn, lt), o.swiglu(g, u), s.ffn, E)
        if not logits:
            return None
        x = o.rmsnorm(h, self.f("output_norm.weight", E), s.eps)
        return o.lm_head(s.embd_type, table, x, E, s.vocab, 0.0)
