"""Seeded synthetic GGUF tensors and activations for the measured workloads.

Block contents (ggml layouts, csrc/gncx_llm_kernels.cpp:266-297):
  Q4_0  fp16 d = |N(0, 0.02)|, 16 bytes of uniform random 4-bit codes
  Q8_0  fp16 d = |N(0, 0.02)|, 32 int8 ~ U[-127, 127]
  Q4_K  fp16 d, dmin = |N(0, 0.02)|, 12 random scale bytes, 128 random nibble bytes
  Q6_K  128 B ql + 64 B qh random, 16 int8 scales ~ U[-32, 31], fp16 d = |N(0, 0.02)|
  BF16  bf16 of N(0, 0.02)
Activations are fp32 N(0, 1).  Everything comes from numpy's PCG64 seeded by
the caller, so the same seed gives the same bytes on every host.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 2, 8, 12, 14, 30
_BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), BF16: (1, 2)}


def _fp16_scales(rng: np.random.Generator, n: int) -> np.ndarray:
    return np.abs(rng.standard_normal(n) * 0.02).astype(np.float16).view(np.uint8).reshape(n, 2)


def make_weights(ggml_type: int, n_rows: int, k: int, seed: int) -> np.ndarray:
    """n_rows x k weights as a flat uint8 array of packed GGUF blocks."""
    be, bb = _BLOCK[ggml_type]
    if k % be:
        raise ValueError(f"k={k} is not a multiple of the block size {be}")
    rng = np.random.default_rng(seed)
    nblk = n_rows * (k // be)
    if ggml_type == BF16:
        w = (rng.standard_normal(n_rows * k) * 0.02).astype(np.float32)
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    out = np.empty((nblk, bb), dtype=np.uint8)
    if ggml_type == Q4_0:
        out[:, 0:2] = _fp16_scales(rng, nblk)
        out[:, 2:18] = rng.integers(0, 256, size=(nblk, 16), dtype=np.uint8)
    elif ggml_type == Q8_0:
        out[:, 0:2] = _fp16_scales(rng, nblk)
        out[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    elif ggml_type == Q4_K:
        out[:, 0:2] = _fp16_scales(rng, nblk)
        out[:, 2:4] = _fp16_scales(rng, nblk)
        out[:, 4:144] = rng.integers(0, 256, size=(nblk, 140), dtype=np.uint8)
    elif ggml_type == Q6_K:
        out[:, 0:192] = rng.integers(0, 256, size=(nblk, 192), dtype=np.uint8)
        out[:, 192:208] = rng.integers(-32, 32, size=(nblk, 16), dtype=np.int8).view(np.uint8)
        out[:, 208:210] = _fp16_scales(rng, nblk)
    else:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    return out.reshape(-1)


def make_activations(rows: int, k: int, seed: int) -> np.ndarray:
    """rows x k fp32 N(0, 1) (flat when rows == 1)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(rows * k).astype(np.float32)
    return x if rows == 1 else x.reshape(rows, k)


def make_norm_gamma(n: int, seed: int) -> np.ndarray:
    """fp32 1 + N(0, 0.1), the norm weights of the attention workloads."""
    rng = np.random.default_rng(seed)
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
