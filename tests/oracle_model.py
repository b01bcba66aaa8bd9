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

    def prefill(self, prompt, progress=None):
        """Logits after the prompt, as the streamer's prefill computes them
        (lua/gncx_streamer.lua:968-1208): per layer, every token's RMSNorm,
        the Q/K/V projections as one matbatch (cpp:1495-1692), each token's
        heads-RMSNorm, RoPE at its position and K/V row, the causal attention
        loop (:1079-1109), then O, the FFN norm, gate/up, SwiGLU and down as
        matbatches with their residual adds.  The caches advance to
        len(prompt), so step() continues the sequence.  In the last layer only
        the final token's row feeds the logits, so O and the FFN run for that
        row alone."""
        o, s = self.o, self.s
        E, lt, B = s.embed, s.layer_type, len(prompt)
        table = self.w("token_embd.weight", s.vocab, E, s.embd_type)
        H = np.stack([o.fetch_embedding(s.embd_type, table, t, E, 1.0) for t in prompt])
        rms_rows = lambda X, g: np.stack([o.rmsnorm(x, g, s.eps) for x in X])  # noqa: E731
        for l in range(s.n_layers):
            p = f"blk.{l}"
            X = rms_rows(H, self.f(f"{p}.attn_norm.weight", E))
            Q = o.matbatch(lt, self.w(f"{p}.attn_q.weight", s.q_dim, E, lt), X, B, E, s.q_dim)
            K = o.matbatch(lt, self.w(f"{p}.attn_k.weight", s.kv_dim, E, lt), X, B, E, s.kv_dim)
            V = o.matbatch(lt, self.w(f"{p}.attn_v.weight", s.kv_dim, E, lt), X, B, E, s.kv_dim)
            gq, gk = self.f(f"{p}.attn_q_norm.weight", s.head_dim), self.f(f"{p}.attn_k_norm.weight", s.head_dim)
            for i in range(B):
                q = o.rmsnorm_heads(Q[i], gq, s.n_heads, s.head_dim, s.eps)
                k = o.rmsnorm_heads(K[i], gk, s.n_kv, s.head_dim, s.eps)
                Q[i], self.kc[l][i] = o.rope(q, k, s.n_heads, s.n_kv, s.head_dim, i, s.rope_base)
                self.vc[l][i] = V[i]
            A = o.attention_prefill(Q, self.kc[l], self.vc[l], 0, B, s.n_heads, s.n_kv, s.head_dim,
                                    1.0 / np.sqrt(s.head_dim), 0)
            if l == s.n_layers - 1:
                A, H = A[-1:], H[-1:]
            n = A.shape[0]
            H = H + o.matbatch(lt, self.w(f"{p}.attn_output.weight", E, s.q_dim, lt), A, n, s.q_dim, E)
            X = rms_rows(H, self.f(f"{p}.ffn_norm.weight", E))
            G = o.matbatch(lt, self.w(f"{p}.ffn_gate.weight", s.ffn, E, lt), X, n, E, s.ffn)
            U = o.matbatch(lt, self.w(f"{p}.ffn_up.weight", s.ffn, E, lt), X, n, E, s.ffn)
            F = np.stack([o.swiglu(g, u) for g, u in zip(G, U)])
            H = H + o.matbatch(lt, self.w(f"{p}.ffn_down.weight", E, s.ffn, lt), F, n, s.ffn, E)
            if progress:
                progress(f"oracle prefill: layer {l + 1}/{s.n_layers} of {B} tokens")
        x = o.rmsnorm(H[-1], self.f("output_norm.weight", E), s.eps)
        return o.lm_head(s.embd_type, table, x, E, s.vocab, 0.0)
