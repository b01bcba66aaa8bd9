"""Qwen3-shaped prefill and decode through the reference C-ABI.

A replay driver: it issues, call for call, what GNCXStreamer:forward_token
(lua/gncx_streamer.lua:759-965) and GNCXStreamer:prefill (:968-1208) issue for
a Qwen3 model (the `is_qwen` branches: per-head Q/K RMSNorm, NEOX RoPE at
`rope_freq_base_global`, attention scale 1/sqrt(head_dim), no sliding window,
SwiGLU, the tied `token_embd.weight` as embedding table and lm_head).  The
differences are where the streamer works on host memory:

* by default every buffer is device memory (torch tensors whose data_ptr()
  goes through the C-ABI, which the library uses in place); with
  Decoder(device="cpu") they are host memory, as in the streamer, and every
  call takes the library's host-pointer path.  host="ram" allocates them as
  the streamer does (lua/gncx_streamer.lua:461-477, 514-564): scratch and
  KV caches from gncx_ram_alloc_colored, the caches coloured by the
  gncx_geo_* slot manager at each layer's gncx_genome_* sieve order; with
  tokens=True the norms and Q/K/V, gate/up and RoPE calls carry the 4-phase
  token array as the streamer's do (lua/gncx_streamer.lua:793-843, 877-891);
* the weights are one device blob laid out like a GGUF data section (tensors
  at 32-byte aligned offsets), addressed as (base, offset) exactly as the
  streamer addresses its mapped file;
* the residual loops (`hidden[i] = hidden[i] + proj_out_buf[i]`,
  lua/gncx_streamer.lua:871-873, 906-908) call gncx_hip_vec_add on device
  buffers and run on the host for host buffers;
* the sampler is a greedy device argmax (the streamer's sampler adds a
  repetition penalty on the host, lua/gncx_streamer.lua:1229-1272);
* `native=True` decodes through gncx_hip_decode_step: the library issues a
  whole token's launches itself (no per-call Python and pointer checks), with
  the residual add + RMSNorm in the prologue of the Q/K/V and gate/up
  launches and SwiGLU in the epilogue of gate/up; decode_greedy() runs steps
  that feed their own device argmax back, with no host round trip per token;
* `fused=True` uses the library's launch-saving extensions, with the same
  results: in decode, gncx_hip_attention_step_fused for the four
  prologue+attention calls, gncx_hip_matvec_multi for Q/K/V and for gate/up
  (one launch each) and gncx_hip_add_rmsnorm for each residual add and the
  RMSNorm after it; in prefill, gncx_hip_fetch_token_embeddings for the
  embedding rows, gncx_hip_matbatch_multi_addnorm for Q/K/V and for gate/up
  with the per-token residual add + RMSNorm loops before them folded in,
  gncx_hip_swiglu_matbatch for the down projection, and
  gncx_hip_attention_prefill for the per-token prologue + attention loop
  (one causal batch).

Weights are random-init with the block statistics of the synthetic
benchmark inputs: fp16 scales |N(0, 0.02)|, uniform random code bytes,
Q6_K sub-block scales U[-32, 31], RMSNorm gammas 1 + N(0, 0.1).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from . import Q4_K, Q6_K, DecodeLayer, DecodeModel, DecodeState, DecodeTensor, row_bytes

_ALIGN = 32  # GGUF default data alignment


@dataclass(frozen=True)
class Qwen3Shape:
    n_layers: int = 36
    embed: int = 4096
    n_heads: int = 32
    n_kv: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 151936
    eps: float = 1e-6
    rope_base: float = 1e6
    layer_type: int = Q4_K
    embd_type: int = Q6_K

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim


QWEN3_8B = Qwen3Shape()


@dataclass
class Model:
    shape: Qwen3Shape
    blob: object  # torch uint8 tensor on the device, or a host mapping of a GGUF file
    offsets: dict = field(default_factory=dict)  # tensor name -> byte offset in blob

    @property
    def base(self) -> int:
        """Address of byte 0: device memory for a torch blob, host memory for
        a mapped GGUF file (the streamer's mmap base, which the library
        uploads from once per tensor)."""
        return self.blob.data_ptr() if hasattr(self.blob, "data_ptr") else self.blob.ctypes.data

    def off(self, name: str) -> int:
        return self.offsets[name]


def _layout(s: Qwen3Shape):
    """(name, kind, rows, cols) in file order; kind is a ggml type or 'f32'."""
    t = [("token_embd.weight", s.embd_type, s.vocab, s.embed)]
    for l in range(s.n_layers):
        p = f"blk.{l}"
        t += [
            (f"{p}.attn_norm.weight", "f32", 1, s.embed),
            (f"{p}.attn_q.weight", s.layer_type, s.q_dim, s.embed),
            (f"{p}.attn_k.weight", s.layer_type, s.kv_dim, s.embed),
            (f"{p}.attn_v.weight", s.layer_type, s.kv_dim, s.embed),
            (f"{p}.attn_q_norm.weight", "f32", 1, s.head_dim),
            (f"{p}.attn_k_norm.weight", "f32", 1, s.head_dim),
            (f"{p}.attn_output.weight", s.layer_type, s.embed, s.q_dim),
            (f"{p}.ffn_norm.weight", "f32", 1, s.embed),
            (f"{p}.ffn_gate.weight", s.layer_type, s.ffn, s.embed),
            (f"{p}.ffn_up.weight", s.layer_type, s.ffn, s.embed),
            (f"{p}.ffn_down.weight", s.layer_type, s.embed, s.ffn),
        ]
    t.append(("output_norm.weight", "f32", 1, s.embed))
    return t


def _nbytes(kind, rows, cols) -> int:
    return 4 * rows * cols if kind == "f32" else row_bytes(kind, cols) * rows


def build_model(torch, shape: Qwen3Shape = QWEN3_8B, seed: int = 0, device: str = "cuda") -> Model:
    """Random-init weights generated on the device into one GGUF-like blob."""
    layout = _layout(shape)
    offsets, total = {}, 0
    for name, kind, rows, cols in layout:
        total = (total + _ALIGN - 1) // _ALIGN * _ALIGN
        offsets[name] = total
        total += _nbytes(kind, rows, cols)
    blob = torch.empty(total, dtype=torch.uint8, device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    for name, kind, rows, cols in layout:
        o, n = offsets[name], _nbytes(kind, rows, cols)
        seg = blob[o:o + n]
        if kind == "f32":
            v = 1.0 + 0.1 * torch.randn(rows * cols, generator=g, device=device)
            seg.view(torch.float32).copy_(v)
            continue
        bb = 144 if kind == Q4_K else 210
        blk = seg.view(-1, bb)
        nb = blk.shape[0]
        blk.copy_(torch.randint(0, 256, (nb, bb), generator=g, device=device, dtype=torch.uint8))
        if kind == Q4_K:  # d, dmin fp16 |N(0, 0.02)|; 12 scale bytes and 128 code bytes stay random
            d = (0.02 * torch.randn(nb, 2, generator=g, device=device)).abs().to(torch.float16)
            blk[:, 0:4].copy_(d.view(torch.uint8).view(nb, 4))
        else:  # Q6_K: 16 int8 scales U[-32, 31] at 192, fp16 d |N(0, 0.02)| at 208
            sc = torch.randint(-32, 32, (nb, 16), generator=g, device=device, dtype=torch.int8)
            blk[:, 192:208].copy_(sc.view(torch.uint8))
            d = (0.02 * torch.randn(nb, 1, generator=g, device=device)).abs().to(torch.float16)
            blk[:, 208:210].copy_(d.view(torch.uint8).view(nb, 2))
    return Model(shape, blob, offsets)


# -- GGUF model files ---------------------------------------------------------
def _gguf_dims(kind, rows, cols):
    return (cols,) if kind == "f32" else (cols, rows)  # ggml order: row length first


def write_model_gguf(path, shape: Qwen3Shape = QWEN3_8B, seed: int = 0) -> dict:
    """A qwen3 GGUF file with the metadata keys the streamer reads
    (lua/gncx_streamer.lua:345-366, 444-451) and random-init tensors with the
    block statistics of build_model, generated on the host one tensor at a
    time.  The vocabulary is `shape.vocab` dummy tokens (the streamer takes
    the vocabulary size from their count).  Returns {name: file offset}."""
    import numpy as np

    from . import gguf as G

    rng = np.random.default_rng(seed)
    a = "qwen3"
    meta = [
        ("general.architecture", G.STRING, a),
        ("general.alignment", G.UINT32, _ALIGN),
        (f"{a}.block_count", G.UINT32, shape.n_layers),
        (f"{a}.context_length", G.UINT32, 40960),
        (f"{a}.embedding_length", G.UINT32, shape.embed),
        (f"{a}.feed_forward_length", G.UINT32, shape.ffn),
        (f"{a}.attention.head_count", G.UINT32, shape.n_heads),
        (f"{a}.attention.head_count_kv", G.UINT32, shape.n_kv),
        (f"{a}.attention.key_length", G.UINT32, shape.head_dim),
        (f"{a}.attention.value_length", G.UINT32, shape.head_dim),
        (f"{a}.attention.layer_norm_rms_epsilon", G.FLOAT32, shape.eps),
        (f"{a}.rope.freq_base", G.FLOAT32, shape.rope_base),
        ("tokenizer.ggml.model", G.STRING, "gpt2"),
        ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, [f"<t{i}>" for i in range(shape.vocab)])),
        ("tokenizer.ggml.token_type", G.ARRAY, (G.INT32, [1] * shape.vocab)),
        ("tokenizer.ggml.merges", G.ARRAY, (G.STRING, [])),
        ("tokenizer.ggml.eos_token_id", G.UINT32, 151645),
    ]

    def writer(kind, rows, cols):
        def w(f):
            if kind == "f32":
                f.write((1.0 + 0.1 * rng.standard_normal(rows * cols)).astype(np.float32).tobytes())
                return
            bb = 144 if kind == Q4_K else 210
            nb_row = row_bytes(kind, cols) // bb
            for r0 in range(0, rows, 1024):  # bounded host memory per chunk
                nb = min(1024, rows - r0) * nb_row
                blk = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
                if kind == Q4_K:
                    blk[:, 0:4] = np.abs(0.02 * rng.standard_normal((nb, 2))).astype(np.float16).view(np.uint8)
                else:
                    blk[:, 192:208] = rng.integers(-32, 32, (nb, 16), dtype=np.int8).view(np.uint8)
                    blk[:, 208:210] = np.abs(0.02 * rng.standard_normal((nb, 1))).astype(np.float16).view(np.uint8)
                f.write(blk.tobytes())
        return w

    specs = []
    for name, kind, rows, cols in _layout(shape):
        t = G.F32 if kind == "f32" else kind
        specs.append(G.TensorSpec(name, t, _gguf_dims(kind, rows, cols), writer(kind, rows, cols)))
    return G.write_gguf(path, meta, specs)


def load_model_gguf(path) -> Model:
    """Map a GGUF file (read-only, host memory) and read the shape from its
    metadata as GNCXStreamer.new does (lua/gncx_streamer.lua:345-366): the
    Model's base is the mapping's address and its offsets the tensors'
    absolute file offsets, so every weight reaches the library as the
    streamer passes it, a host pointer (base, offset)."""
    import numpy as np

    from . import gguf as G

    mm = np.memmap(path, dtype=np.uint8, mode="r")
    meta, tensors, _ = G.read_gguf(mm)
    a = meta.get("general.architecture", "qwen3")
    n_heads = int(meta[f"{a}.attention.head_count"])
    embed = int(meta[f"{a}.embedding_length"])
    shape = Qwen3Shape(
        n_layers=int(meta[f"{a}.block_count"]), embed=embed, n_heads=n_heads,
        n_kv=int(meta.get(f"{a}.attention.head_count_kv", n_heads)),
        head_dim=int(meta.get(f"{a}.attention.key_length", embed // n_heads)),
        ffn=int(meta[f"{a}.feed_forward_length"]), vocab=len(meta.get("tokenizer.ggml.tokens", [])),
        eps=float(meta.get(f"{a}.attention.layer_norm_rms_epsilon", 1e-6)),
        rope_base=float(meta.get(f"{a}.rope.freq_base", 10000.0)),
        layer_type=tensors["blk.0.attn_q.weight"].ggml_type, embd_type=tensors["token_embd.weight"].ggml_type)
    return Model(shape, mm, {n: t.abs_file_offset for n, t in tensors.items()})


class Decoder:
    """State of one sequence and the streamer's call sequence.  device="cuda"
    keeps every buffer in device memory (the library uses them in place);
    device="cpu" keeps them in host memory as the streamer does (its buffers
    and KV caches are host RAM), so every call goes through the library's
    host-pointer path: inputs staged, outputs written back before return, KV
    caches mirrored by device twins, residual adds on the host."""

    def __init__(self, lib, torch, model: Model, max_seq: int, fused: bool = False, device: str = "cuda",
                 native: bool = False, host: str = "torch", tokens: bool = False, layer_k: int = 3,
                 driver: str = "python"):
        s = model.shape
        self.lib, self.torch, self.m, self.s, self.fused, self.native = lib, torch, model, s, fused, native
        if native and device != "cuda":
            raise ValueError("the native decode step keeps every buffer in device memory")
        if host == "ram" and device != "cpu":
            raise ValueError("host='ram' places the buffers in host memory: device must be 'cpu'")
        f32 = dict(dtype=torch.float32, device=device)
        self._ram = []  # gncx_ram_* handles, freed by close()
        if host == "ram":
            import numpy as np

            def buf(n, slot_d, k=1, r=3, rows=None):
                count = n * (rows or 1)
                h = lib.gncx_ram_alloc_colored(max(count * 4, 4096), k, slot_d, r)
                if not h:
                    raise MemoryError("gncx_ram_alloc_colored failed")
                self._ram.append(h)
                a = np.ctypeslib.as_array((C.c_float * count).from_address(lib.gncx_ram_get_ptr(h)))
                t = torch.from_numpy(a)
                return t.view(rows, n) if rows else t
        else:
            def buf(n, slot_d, k=1, r=3, rows=None):
                return torch.zeros(*((rows, n) if rows else (n,)), **f32)
        # the streamer's scratch colours (lua/gncx_streamer.lua:461-477)
        self.hidden = buf(s.embed, 0)
        self.normed = buf(s.embed, 1)
        self.q = buf(s.q_dim, 2)
        self.k = buf(s.kv_dim, 3)
        self.v = buf(s.kv_dim, 4)
        self.attn = buf(s.q_dim, 5)
        self.proj = buf(s.embed, 6)
        self.gate = buf(s.ffn, 7)
        self.up = buf(s.ffn, 8)
        self.act = buf(s.ffn, 9)
        self.logits = buf(s.vocab, 10)
        # per-layer sieve order (lua/gncx_streamer.lua:502-511)
        self.crivo = []
        out = [C.c_int32() for _ in range(4)]
        for l in range(s.n_layers):
            lib.gncx_genome_get_layer_coordinate(l, s.n_layers, layer_k, *[C.addressof(o) for o in out])
            self.crivo.append(out[2].value)
        self.layer_k = layer_k
        self.kc, self.vc = [], []
        if host == "ram":
            # KV caches coloured by the slot manager (lua/gncx_streamer.lua:514-564)
            gmm = lib.gncx_geo_mm_create(s.n_layers * 2)
            kk, dd, rr, idx = C.c_uint8(), C.c_uint8(), C.c_uint8(), C.c_uint32()
            try:
                for l in range(s.n_layers):
                    for lst in (self.kc, self.vc):
                        lib.gncx_geo_alloc(gmm, self.crivo[l], C.addressof(kk), C.addressof(dd), C.addressof(rr),
                                           C.addressof(idx))
                        lst.append(buf(s.kv_dim, dd.value, kk.value, rr.value, rows=max_seq))
            finally:
                lib.gncx_geo_mm_destroy(gmm)
        else:
            self.kc = [buf(s.kv_dim, 0, rows=max_seq) for _ in range(s.n_layers)]
            self.vc = [buf(s.kv_dim, 0, rows=max_seq) for _ in range(s.n_layers)]
        # the 4-phase token array and quant scale (lua/gncx_streamer.lua:486-487)
        from . import GNCXCompactToken
        self.tokens = (GNCXCompactToken * max(s.embed, s.q_dim, s.ffn))() if tokens else None
        self.qscale = (C.c_float * 1)()
        if driver not in ("python", "c"):
            raise ValueError("driver is 'python' or 'c'")
        self.driver, self._replay = driver, None
        self.max_seq = max_seq
        self.scale = 1.0 / (s.head_dim ** 0.5)
        self._qkv = self._gu = None  # gncx_hip_matvec_multi arguments, built on first fused use
        self._native = None  # gncx_hip_decode_step structs, built on first native use

    def _add(self, dst, src):
        """hidden += delta: the streamer's host loop (lua/gncx_streamer.lua:871-873,
        906-908) for host buffers, gncx_hip_vec_add for device ones."""
        if dst.is_cuda:
            self.lib.gncx_hip_vec_add(dst.data_ptr(), src.data_ptr(), dst.numel())
        else:
            dst += src

    def _fused_tables(self):
        """ctypes argument arrays of gncx_hip_matvec_multi, per layer."""
        s, m = self.s, self.m
        P, I = C.c_void_p, C.c_int32
        self._qkv, self._gu = [], []
        for l in range(s.n_layers):
            p = f"blk.{l}"
            w = (P * 3)(*(m.base + m.off(f"{p}.attn_{n}.weight") for n in "qkv"))
            y = (P * 3)(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr())
            self._qkv.append((w, (I * 3)(s.q_dim, s.kv_dim, s.kv_dim), y))
            w = (P * 2)(m.base + m.off(f"{p}.ffn_gate.weight"), m.base + m.off(f"{p}.ffn_up.weight"))
            y = (P * 2)(self.gate.data_ptr(), self.up.data_ptr())
            self._gu.append((w, (I * 2)(s.ffn, s.ffn), y))

    # -- the pieces shared by forward_token and prefill ----------------------
    def close(self):
        """Free the gncx_ram_* buffers (host="ram"); the buffers' tensors must
        not be used afterwards."""
        for h in self._ram:
            self.lib.gncx_ram_free(h)
        self._ram = []

    def _tok(self):
        return C.addressof(self.tokens) if self.tokens is not None else None

    def _matvec(self, name, x, in_dim, out_dim, y, tokens=None):
        self.lib.gncx_xfold_universal_matvec(self.m.base, self.m.off(name), self.s.layer_type, x, tokens, in_dim,
                                             out_dim, y, None)

    def _matbatch(self, name, x, b, in_dim, out_dim, y):
        self.lib.gncx_xfold_universal_matbatch(self.m.base, self.m.off(name), self.s.layer_type, x, b, in_dim,
                                               out_dim, y, None)

    def _norm(self, name, x, out, layer_k=0):
        tk = self._tok()
        self.lib.gncx_rmsnorm_and_encode_4phase(x, self.m.base, self.m.off(name), self.s.embed, self.s.eps, layer_k,
                                                out, tk, C.addressof(self.qscale) if tk else None)

    def _attention(self, l, q, k, v, pos, out):
        s, L, m = self.s, self.lib, self.m
        p = f"blk.{l}"
        kc, vc = self.kc[l].data_ptr(), self.vc[l].data_ptr()
        if self.fused:
            L.gncx_hip_attention_step_fused(q, k, v, kc, vc, pos, s.n_heads, s.n_kv, s.head_dim, self.scale, 0, 1,
                                            m.base, m.off(f"{p}.attn_q_norm.weight"),
                                            m.off(f"{p}.attn_k_norm.weight"), 1, s.eps, 0, 0, s.rope_base, out)
            return
        L.gncx_rmsnorm_inplace_heads(q, m.base, m.off(f"{p}.attn_q_norm.weight"), 1, s.n_heads, s.head_dim, s.eps)
        L.gncx_rmsnorm_inplace_heads(k, m.base, m.off(f"{p}.attn_k_norm.weight"), 1, s.n_kv, s.head_dim, s.eps)
        L.gncx_apply_rope_xor11_ext(q, k, self._tok(), None, 0, 0, s.n_heads, s.n_kv, s.head_dim, pos, s.rope_base)
        L.gncx_mqa_attention_step_ext(q, k, v, kc, vc, pos, s.n_heads, s.n_kv, s.head_dim, self.scale, 0, 1, out)

    def _lm_head(self, normed_ready: bool = False):
        s, m = self.s, self.m
        if not normed_ready:
            self._norm("output_norm.weight", self.hidden.data_ptr(), self.normed.data_ptr(), self.layer_k)
        self.lib.gncx_universal_lm_head_logits(m.base, m.off("token_embd.weight"), s.embd_type,
                                               self.normed.data_ptr(), s.embed, s.vocab, 0.0,
                                               self.logits.data_ptr())
        return self.logits

    def _embed(self, token, dst):
        s, m = self.s, self.m
        fetch = {Q6_K: self.lib.gncx_fetch_token_embedding_q6_k}[s.embd_type]
        fetch(m.base, m.off("token_embd.weight"), int(token), s.embed, 1.0, dst)

    # -- the native decode step ---------------------------------------------------
    def _native_structs(self):
        torch, s, m = self.torch, self.s, self.m
        T = lambda name, kind=None: DecodeTensor(m.off(name), s.layer_type if kind is None else kind)  # noqa: E731
        layers = (DecodeLayer * s.n_layers)()
        for l in range(s.n_layers):
            p = f"blk.{l}"
            layers[l] = DecodeLayer(T(f"{p}.attn_norm.weight", -1), T(f"{p}.attn_q.weight"), T(f"{p}.attn_k.weight"),
                                    T(f"{p}.attn_v.weight"), T(f"{p}.attn_q_norm.weight", -1),
                                    T(f"{p}.attn_k_norm.weight", -1), T(f"{p}.attn_output.weight"),
                                    T(f"{p}.ffn_norm.weight", -1), T(f"{p}.ffn_gate.weight"),
                                    T(f"{p}.ffn_up.weight"), T(f"{p}.ffn_down.weight"))
        model = DecodeModel(m.base, layers, T("token_embd.weight", s.embd_type), T("output_norm.weight", -1),
                            s.n_layers, s.embed, s.n_heads, s.n_kv, s.head_dim, s.ffn, s.vocab, 1, s.eps,
                            s.rope_base, self.scale)
        f32 = dict(dtype=torch.float32, device=self.hidden.device)
        self.hidden2 = torch.zeros(s.embed, **f32)
        self.token_dev = torch.zeros(1, dtype=torch.int32, device=self.hidden.device)
        self.token_log = torch.full((self.max_seq,), -1, dtype=torch.int32, device=self.hidden.device)
        P = C.c_void_p
        kc = (P * s.n_layers)(*(t.data_ptr() for t in self.kc))
        vc = (P * s.n_layers)(*(t.data_ptr() for t in self.vc))
        state = DecodeState((P * 2)(self.hidden.data_ptr(), self.hidden2.data_ptr()), self.q.data_ptr(),
                            self.k.data_ptr(), self.v.data_ptr(), self.attn.data_ptr(), self.proj.data_ptr(),
                            self.normed.data_ptr(), self.gate.data_ptr(), self.up.data_ptr(), self.act.data_ptr(),
                            self.logits.data_ptr(), C.cast(kc, C.POINTER(P)), C.cast(vc, C.POINTER(P)),
                            self.max_seq, self.token_dev.data_ptr(), self.token_log.data_ptr())
        self._native = (layers, model, kc, vc, state)

    def _step(self, token: int, pos: int, greedy: bool):
        if pos < 0 or pos >= self.max_seq:
            raise ValueError("position past the KV cache")
        if self._native is None:
            self._native_structs()
        _, model, _, _, state = self._native
        if self.lib.gncx_hip_decode_step(C.byref(model), C.byref(state), int(token), int(pos), int(greedy)) != 0:
            raise RuntimeError(self.lib.gncx_hip_last_error().decode())

    def decode_greedy(self, token: int, pos: int, n: int) -> list:
        """n greedy steps from `token` at `pos` through the native step: each
        step's device argmax is the next step's input token, and the host waits
        once, for the n chosen tokens (the streamer's sampler, without its
        repetition penalty, lua/gncx_streamer.lua:1229-1272)."""
        for i in range(n):
            self._step(token if i == 0 else -1, pos + i, True)
        return self.token_log[pos:pos + n].tolist()

    # -- lua/gncx_streamer.lua:759-965 ------------------------------------------
    def _replay_token(self, token: int, pos: int):
        """forward_token issued from native code (gnc-x_amd/bin/gncx_streamer_replay.so)."""
        if self._replay is None:
            from . import LIB_PATH, GNCXTelemetryStats
            if self._native is None:
                self._native_structs()
            so = C.CDLL(str(LIB_PATH.parent / "gncx_streamer_replay.so"))
            fn = so.gncx_replay_forward_token
            fn.restype = C.c_int
            fn.argtypes = [C.c_void_p] * 6 + [C.c_int32] * 4
            self._replay = (so, fn, (C.c_int32 * self.s.n_layers)(*self.crivo), GNCXTelemetryStats())
        _, fn, crivo, tel = self._replay
        _, model, _, _, state = self._native
        tk = C.addressof(self.tokens) if self.tokens is not None else None
        rc = fn(C.addressof(model), C.addressof(state), tk, C.addressof(self.qscale), C.addressof(tel),
                C.addressof(crivo), self.layer_k, int(token), int(pos), 1)
        if rc != 0:
            raise RuntimeError(self.lib.gncx_hip_last_error().decode())
        return self.logits

    def forward_token(self, token: int, pos: int):
        s, L = self.s, self.lib
        if pos >= self.max_seq:
            raise ValueError("position past the KV cache")
        if self.native:
            self._step(token, pos, False)
            return self.logits
        if self.driver == "c":
            return self._replay_token(token, pos)
        h, nrm = self.hidden.data_ptr(), self.normed.data_ptr()
        q, k, v, a = self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.attn.data_ptr()
        pr, ga, up, ac = self.proj.data_ptr(), self.gate.data_ptr(), self.up.data_ptr(), self.act.data_ptr()
        self._embed(token, h)
        if self.fused:
            return self._forward_fused(pos)
        tk = self._tok()
        for l in range(s.n_layers):
            p = f"blk.{l}"
            self._norm(f"{p}.attn_norm.weight", h, nrm, self.crivo[l])
            self._matvec(f"{p}.attn_q.weight", nrm, s.embed, s.q_dim, q, tk)
            self._matvec(f"{p}.attn_k.weight", nrm, s.embed, s.kv_dim, k, tk)
            self._matvec(f"{p}.attn_v.weight", nrm, s.embed, s.kv_dim, v, tk)
            self._attention(l, q, k, v, pos, a)
            self._matvec(f"{p}.attn_output.weight", a, s.q_dim, s.embed, pr)
            self._add(self.hidden, self.proj)
            self._norm(f"{p}.ffn_norm.weight", h, nrm, self.crivo[l])
            self._matvec(f"{p}.ffn_gate.weight", nrm, s.embed, s.ffn, ga, tk)
            self._matvec(f"{p}.ffn_up.weight", nrm, s.embed, s.ffn, up, tk)
            L.gncx_swiglu_activation(ga, up, s.ffn, ac)
            self._matvec(f"{p}.ffn_down.weight", ac, s.ffn, s.embed, pr)
            self._add(self.hidden, self.proj)
        return self._lm_head()

    def _forward_fused(self, pos: int):
        """forward_token's layers with the extensions: 8 calls per layer."""
        s, L, m = self.s, self.lib, self.m
        h, nrm = self.hidden.data_ptr(), self.normed.data_ptr()
        q, k, v, a = self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.attn.data_ptr()
        pr, ga, up, ac = self.proj.data_ptr(), self.gate.data_ptr(), self.up.data_ptr(), self.act.data_ptr()
        if self._qkv is None:
            self._fused_tables()
        self._norm("blk.0.attn_norm.weight", h, nrm)
        for l in range(s.n_layers):
            p = f"blk.{l}"
            w, n, y = self._qkv[l]
            L.gncx_hip_matvec_multi(3, w, n, s.layer_type, nrm, s.embed, y)
            self._attention(l, q, k, v, pos, a)
            self._matvec(f"{p}.attn_output.weight", a, s.q_dim, s.embed, pr)
            L.gncx_hip_add_rmsnorm(h, pr, m.base, m.off(f"{p}.ffn_norm.weight"), s.embed, s.eps, nrm)
            w, n, y = self._gu[l]
            L.gncx_hip_matvec_multi(2, w, n, s.layer_type, nrm, s.embed, y)
            L.gncx_swiglu_activation(ga, up, s.ffn, ac)
            self._matvec(f"{p}.ffn_down.weight", ac, s.ffn, s.embed, pr)
            nxt = f"blk.{l + 1}.attn_norm.weight" if l + 1 < s.n_layers else "output_norm.weight"
            L.gncx_hip_add_rmsnorm(h, pr, m.base, m.off(nxt), s.embed, s.eps, nrm)
        return self._lm_head(normed_ready=True)

    # -- lua/gncx_streamer.lua:968-1208 -----------------------------------------
    def prefill(self, token_ids):
        torch, s, L = self.torch, self.s, self.lib
        B = len(token_ids)
        if B == 0:
            return None
        if B == 1:
            return self.forward_token(token_ids[0], 0)
        if B > self.max_seq:
            raise ValueError("prompt longer than the KV cache")
        f32 = dict(dtype=torch.float32, device=self.hidden.device)
        bh = torch.zeros(B, s.embed, **f32)
        bn = torch.zeros(B, s.embed, **f32)
        bq = torch.zeros(B, s.q_dim, **f32)
        bk = torch.zeros(B, s.kv_dim, **f32)
        bv = torch.zeros(B, s.kv_dim, **f32)
        ba = torch.zeros(B, s.q_dim, **f32)
        bp = torch.zeros(B, s.embed, **f32)
        bg = torch.zeros(B, s.ffn, **f32)
        bu = torch.zeros(B, s.ffn, **f32)
        bf = torch.zeros(B, s.ffn, **f32)
        rowp = lambda t, i: t.data_ptr() + 4 * i * t.shape[1]  # noqa: E731
        if self.fused:
            ids = (C.c_int32 * B)(*(int(t) for t in token_ids))
            L.gncx_hip_fetch_token_embeddings(s.embd_type, self.m.base, self.m.off("token_embd.weight"), ids, B,
                                              s.vocab, s.embed, 1.0, bh.data_ptr())
            return self._prefill_fused(B, bh, bn, bq, bk, bv, ba, bp, bg, bu, bf)
        for i, tok in enumerate(token_ids):
            self._embed(tok, rowp(bh, i))
        for l in range(s.n_layers):
            p = f"blk.{l}"
            for i in range(B):
                self._norm(f"{p}.attn_norm.weight", rowp(bh, i), rowp(bn, i))
            self._matbatch(f"{p}.attn_q.weight", bn.data_ptr(), B, s.embed, s.q_dim, bq.data_ptr())
            self._matbatch(f"{p}.attn_k.weight", bn.data_ptr(), B, s.embed, s.kv_dim, bk.data_ptr())
            self._matbatch(f"{p}.attn_v.weight", bn.data_ptr(), B, s.embed, s.kv_dim, bv.data_ptr())
            for i in range(B):
                self._attention(l, rowp(bq, i), rowp(bk, i), rowp(bv, i), i, rowp(ba, i))
            self._matbatch(f"{p}.attn_output.weight", ba.data_ptr(), B, s.q_dim, s.embed, bp.data_ptr())
            self._add(bh, bp)
            for i in range(B):
                self._norm(f"{p}.ffn_norm.weight", rowp(bh, i), rowp(bn, i))
            self._matbatch(f"{p}.ffn_gate.weight", bn.data_ptr(), B, s.embed, s.ffn, bg.data_ptr())
            self._matbatch(f"{p}.ffn_up.weight", bn.data_ptr(), B, s.embed, s.ffn, bu.data_ptr())
            L.gncx_swiglu_activation(bg.data_ptr(), bu.data_ptr(), B * s.ffn, bf.data_ptr())
            self._matbatch(f"{p}.ffn_down.weight", bf.data_ptr(), B, s.ffn, s.embed, bp.data_ptr())
            self._add(bh, bp)
        self.hidden.copy_(bh[B - 1])
        return self._lm_head()

    def _prefill_fused(self, B, bh, bn, bq, bk, bv, ba, bp, bg, bu, bf):
        """prefill's layers with the extensions: every token's RMSNorm (with
        the residual add before it) inside the next matbatch's activation
        pass (gncx_hip_matbatch_multi_addnorm), the per-token prologue +
        attention loop as one causal batch (gncx_hip_attention_prefill), and
        the SwiGLU inside the down projection's matbatch."""
        s, L, m = self.s, self.lib, self.m
        self._norm_rows = bn
        for l in range(s.n_layers):
            p = f"blk.{l}"
            # the previous layer's residual add and this layer's first norm go
            # into the Q/K/V matbatch's activation pass
            self._matbatch_multi_addnorm(p, "qkv", "attn_norm", bh, None if l == 0 else bp, B,
                                         (s.q_dim, s.kv_dim, s.kv_dim), (bq, bk, bv))
            L.gncx_hip_attention_prefill(bq.data_ptr(), bk.data_ptr(), bv.data_ptr(), self.kc[l].data_ptr(),
                                         self.vc[l].data_ptr(), 0, B, s.n_heads, s.n_kv, s.head_dim, self.scale, 0,
                                         m.base, m.off(f"{p}.attn_q_norm.weight"), m.off(f"{p}.attn_k_norm.weight"),
                                         1, s.eps, 0, 0, s.rope_base, ba.data_ptr())
            self._matbatch(f"{p}.attn_output.weight", ba.data_ptr(), B, s.q_dim, s.embed, bp.data_ptr())
            self._matbatch_multi_addnorm(p, ("ffn_gate", "ffn_up"), "ffn_norm", bh, bp, B, (s.ffn, s.ffn), (bg, bu))
            # SwiGLU formed by the down projection's activation pass
            L.gncx_hip_swiglu_matbatch(m.base, m.off(f"{p}.ffn_down.weight"), s.layer_type, bg.data_ptr(),
                                       bu.data_ptr(), B, s.ffn, s.embed, bp.data_ptr())
        self._add(bh, bp)
        self.hidden.copy_(bh[B - 1])
        return self._lm_head()

    def _matbatch_multi_addnorm(self, p, names, norm, hidden, delta, b, out_dims, outs):
        """gncx_hip_matbatch_multi_addnorm: hidden += delta (None: no add), then
        the matrices {p}.{name}.weight applied to the RMSNorm ({p}.{norm}.weight)
        of the rows; on host buffers the two calls it fuses, the rows normed
        into the prefill's norm buffer."""
        P, I = C.c_void_p, C.c_int32
        if names == "qkv":
            names = ("attn_q", "attn_k", "attn_v")
        n = len(names)
        w = (P * n)(*(self.m.base + self.m.off(f"{p}.{nm}.weight") for nm in names))
        y = (P * n)(*(t.data_ptr() for t in outs))
        if not hidden.is_cuda:
            # host buffers (the entry takes device memory): the two calls it fuses
            L, g, bn = self.lib, self.m.off(f"{p}.{norm}.weight"), self._norm_rows
            if delta is None:
                L.gncx_hip_rmsnorm_rows(hidden.data_ptr(), b, self.m.base, g, self.s.embed, self.s.eps,
                                        bn.data_ptr())
            else:
                L.gncx_hip_add_rmsnorm_rows(hidden.data_ptr(), delta.data_ptr(), b, self.m.base, g, self.s.embed,
                                            self.s.eps, bn.data_ptr())
            L.gncx_hip_matbatch_multi(n, w, (I * n)(*out_dims), self.s.layer_type, bn.data_ptr(), b, self.s.embed, y)
            return
        self.lib.gncx_hip_matbatch_multi_addnorm(hidden.data_ptr(), None if delta is None else delta.data_ptr(),
                                                 self.m.base, self.m.off(f"{p}.{norm}.weight"), self.s.eps, n, w,
                                                 (I * n)(*out_dims), self.s.layer_type, b, self.s.embed, y)

    def greedy(self, logits) -> int:
        return int(self.torch.argmax(logits).item())

    def generate(self, prompt, n_new: int):
        """Prefill `prompt`, then n_new greedy decode steps; returns the new ids."""
        out = []
        logits = self.prefill(list(prompt))
        pos = len(prompt)
        for _ in range(n_new):
            tok = self.greedy(logits)
            out.append(tok)
            logits = self.forward_token(tok, pos)
            pos += 1
        return out
