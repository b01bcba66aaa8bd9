"""gncx_amd -- Python (ctypes) view of the MI355X-native gncx_llm_core.so.

The product is the C-ABI shared library built from ``csrc/`` into
``bin/gncx_llm_core.so``; it exports the reference's entry points with the
reference's signatures (csrc/gncx_llm_kernels.cpp of GNC-X, bound by LuaJIT
FFI in lua/gncx_streamer.lua:16-252) plus a few ``gncx_hip_*`` extensions.
This module only declares those signatures for ctypes callers (the tests and
bench.py), the way the reference's own ctypes test binds its library
(verify_gncx_fixes.py:61-119).  There is no Python or CPU compute path here:
``load()`` raises if the library has not been built.

The directory is named ``gnc-x_amd``; import it as ``gncx_amd`` through
:func:`import_from` (a dash cannot appear in a Python module name).
"""
from __future__ import annotations

import ctypes as C
import importlib.util
import os
import pathlib
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "bin" / "gncx_llm_core.so"
CSRC_DIR = PKG_DIR / "csrc"

# ggml type ids (csrc/gncx_llm_kernels.cpp:1362-1462)
Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 2, 8, 12, 14, 30
TYPE_NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", BF16: "BF16"}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256, BF16: 1}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210, BF16: 2}


def row_bytes(ggml_type: int, k: int) -> int:
    """Bytes of one row of k weights (whole blocks only, like the reference)."""
    return (k // BLOCK_ELEMS[ggml_type]) * BLOCK_BYTES[ggml_type]


class GNCXCompactToken(C.Structure):
    """cpp:267-271 (packed, 4 bytes)."""

    _pack_ = 1
    _fields_ = [("phase_2bit", C.c_uint8), ("diag_d", C.c_uint8), ("abs_delta", C.c_uint16)]


class GNCXTelemetryStats(C.Structure):
    """cpp:308-313 (packed, 4 x u64)."""

    _pack_ = 1
    _fields_ = [
        ("total_macs_equivalent", C.c_uint64),
        ("zero_origin_cancellations", C.c_uint64),
        ("zero_weight_skips", C.c_uint64),
        ("xfold_bucket_merges", C.c_uint64),
    ]


_vp, _fp, _i32, _f32, _sz = C.c_void_p, C.c_void_p, C.c_int32, C.c_float, C.c_size_t

# name -> (restype, argtypes); pointers are passed as integers (host or device)
SIGNATURES = {
    # reference entry points
    "gncx_xfold_universal_matvec": (None, [_vp, _sz, _i32, _fp, _vp, _i32, _i32, _fp, _vp]),
    "gncx_xfold_q4_0_matvec": (None, [_vp, _sz, _fp, _vp, _i32, _i32, _fp, _vp]),
    "gncx_xfold_universal_matbatch": (None, [_vp, _sz, _i32, _fp, _i32, _i32, _i32, _fp, _vp]),
    "gncx_xfold_q4_0_matbatch": (None, [_vp, _sz, _fp, _i32, _i32, _i32, _fp, _vp]),
    "gncx_universal_lm_head_logits": (None, [_vp, _sz, _i32, _fp, _i32, _i32, _f32, _fp]),
    "gncx_q8_0_lm_head_logits": (None, [_vp, _sz, _fp, _i32, _i32, _fp]),
    "gncx_mqa_attention_step_ext": (None, [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _fp]),
    "gncx_mqa_attention_step": (None, [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32, _fp]),
    "gncx_rmsnorm_inplace_heads": (None, [_fp, _vp, _sz, _i32, _i32, _i32, _f32]),
    "gncx_apply_rope_xor11_ext": (None, [_fp, _fp, _vp, _vp, _sz, _i32, _i32, _i32, _i32, _i32, _f32]),
    "gncx_apply_rope_xor11": (None, [_fp, _fp, _vp, _i32, _i32, _i32, _i32, _f32]),
    "gncx_rmsnorm_and_encode_4phase": (None, [_fp, _vp, _sz, _i32, _f32, _i32, _fp, _vp, _fp]),
    "gncx_swiglu_activation": (None, [_fp, _fp, _i32, _fp]),
    "gncx_fetch_token_embedding_q8_0": (None, [_vp, _sz, _i32, _i32, _f32, _fp]),
    "gncx_fetch_token_embedding_q6_k": (None, [_vp, _sz, _i32, _i32, _f32, _fp]),
    "gncx_fetch_token_embedding_bf16": (None, [_vp, _sz, _i32, _i32, _f32, _fp]),
    "gncx_geglu_activation": (None, [_fp, _fp, _i32, _fp]),
    "gncx_gla_map_readonly": (_vp, [C.c_char_p, _vp]),
    "gncx_gla_get_base_ptr": (_vp, [_vp]),
    "gncx_gla_unmap": (None, [_vp]),
    "gncx_gla_prefetch_range": (None, [_vp, _sz, _sz]),
    "gncx_ram_alloc_colored": (_vp, [_sz, C.c_uint8, C.c_uint8, C.c_uint8]),
    "gncx_ram_alloc": (_vp, [_sz]),
    "gncx_ram_get_ptr": (_vp, [_vp]),
    "gncx_ram_get_ddr3_bank": (C.c_uint8, [_vp]),
    "gncx_ram_get_l1_set": (C.c_uint8, [_vp]),
    "gncx_ram_free": (None, [_vp]),
    "gncx_ram_copy_chunk": (None, [_vp, _sz, _vp, _sz, _sz]),
    "gncx_genome_get_layer_coordinate": (None, [_i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "gncx_geo_mm_create": (_vp, [C.c_uint32]),
    "gncx_geo_mm_destroy": (None, [_vp]),
    "gncx_geo_alloc": (_i32, [_vp, C.c_uint8, _vp, _vp, _vp, _vp]),
    "gncx_geo_free": (None, [_vp, C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint32]),
    "gncx_geo_fragmentation": (_f32, [_vp]),
    "gncx_geo_used": (_sz, [_vp]),
    "gncx_geo_capacity": (_sz, [_vp]),
    # exported but not provided (a call records an error, outputs untouched)
    "gncx_lora_init_adapter": (None, [_fp, _fp, _i32, _i32, _i32, C.c_uint64]),
    "gncx_lora_forward_add": (None, [_fp, _fp, _fp, _i32, _i32, _i32, _f32, _fp]),
    "gncx_lora_backward_step": (None, [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _f32, _f32, _f32]),
    "gncx_mezo_perturb_params": (None, [_fp, _i32, C.c_uint64, _f32]),
    "gncx_mezo_update_params": (None, [_fp, _i32, C.c_uint64, _f32, _f32, _f32]),
    "gncx_cross_entropy_loss": (_f32, [_fp, _i32, _i32, _fp]),
    "gncx_project_layer_3d_point": (None, [_i32, _i32, _vp, _fp, _i32, _vp]),
    "gncx_cosine_similarity": (_f32, [_fp, _fp, _i32]),
    "gncx_vector_l2_normalize": (None, [_fp, _i32]),
    "gncx_mean_pooling": (None, [_fp, _i32, _i32, _fp]),
    "gncx_bidirectional_attention_gqa": (None, [_fp, _fp, _fp, _i32, _i32, _i32, _i32, _f32, _fp]),
    "gncx_bidirectional_attention": (None, [_fp, _fp, _fp, _i32, _i32, _i32, _f32, _fp]),
    # extensions
    "gncx_hip_init": (C.c_int, [C.c_int]),
    "gncx_hip_set_stream": (None, [_vp]),
    "gncx_hip_get_stream": (_vp, []),
    "gncx_hip_synchronize": (C.c_int, []),
    "gncx_hip_last_error": (C.c_char_p, []),
    "gncx_hip_last_status": (C.c_int, []),
    "gncx_hip_weight_forget": (None, [_vp]),
    "gncx_hip_kv_forget": (None, [_fp]),
    "gncx_hip_weight_bytes": (C.c_size_t, []),
    "gncx_hip_dequantize": (None, [_vp, _sz, _i32, _i32, _i32, _fp]),
    "gncx_hip_quantize_act": (None, [_fp, _i32, _i32, _vp, _vp]),
    "gncx_hip_vec_add": (None, [_fp, _fp, _i32]),
    "gncx_hip_matvec_multi": (None, [_i32, _vp, _vp, _i32, _fp, _i32, _vp]),
    "gncx_hip_matbatch_multi": (None, [_i32, _vp, _vp, _i32, _fp, _i32, _i32, _vp]),
    "gncx_hip_fetch_token_embeddings": (None, [_i32, _vp, _sz, _vp, _i32, _i32, _i32, _f32, _fp]),
    "gncx_hip_add_rmsnorm": (None, [_fp, _fp, _vp, _sz, _i32, _f32, _fp]),
    "gncx_hip_add_rmsnorm_rows": (None, [_fp, _fp, _i32, _vp, _sz, _i32, _f32, _fp]),
    "gncx_hip_swiglu_matbatch": (None, [_vp, _sz, _i32, _fp, _fp, _i32, _i32, _i32, _fp]),
    "gncx_hip_attention_prefill": (
        None,
        [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp, _sz, _sz, _i32, _f32, _sz, _i32,
         _f32, _fp],
    ),
    "gncx_hip_rmsnorm_rows": (None, [_fp, _i32, _vp, _sz, _i32, _f32, _fp]),
    "gncx_hip_attention_step_fused": (
        None,
        [_fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp, _sz, _sz, _i32, _f32, _sz, _i32,
         _f32, _fp],
    ),
    "gncx_hip_matvec_multi_addnorm": (None, [_fp, _fp, _vp, _sz, _f32, _fp, _i32, _vp, _vp, _i32, _i32, _vp]),
    "gncx_hip_matbatch_multi_addnorm": (None, [_fp, _fp, _vp, _sz, _f32, _i32, _vp, _vp, _i32, _i32, _i32, _vp]),
    "gncx_hip_matvec_swiglu": (None, [_vp, _vp, _i32, _fp, _i32, _i32, _fp]),
    "gncx_hip_decode_step": (C.c_int, [_vp, _vp, _i32, _i32, _i32]),
    "gncx_hip_decode_step_noalloc": (C.c_int, [_vp, _vp, _i32, _i32, _i32]),
    "gncx_hip_argmax": (None, [_fp, _i32, _vp]),
    "gncx_hip_set_host_coherence": (C.c_int, [C.c_int]),
    "gncx_hip_host_flush": (None, [_vp]),
}


# ctypes mirrors of the native decode step's structs (include/gncx_llm_core.h)
class DecodeTensor(C.Structure):
    _fields_ = [("offset", C.c_size_t), ("ggml_type", C.c_int32)]


class DecodeLayer(C.Structure):
    _fields_ = [(n, DecodeTensor) for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_q_norm", "attn_k_norm",
                                            "attn_output", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")]


class DecodeModel(C.Structure):
    _fields_ = [("base", C.c_void_p), ("layers", C.POINTER(DecodeLayer)), ("token_embd", DecodeTensor),
                ("output_norm", DecodeTensor)] + \
               [(n, C.c_int32) for n in ("n_layers", "embed", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                                         "qk_norm")] + \
               [("eps", C.c_float), ("rope_base", C.c_float), ("attn_scale", C.c_float)]


class DecodeState(C.Structure):
    _fields_ = [("hidden", C.c_void_p * 2)] + \
               [(n, C.c_void_p) for n in ("q", "k", "v", "attn", "proj", "normed", "gate", "up", "act", "logits")] + \
               [("k_cache", C.POINTER(C.c_void_p)), ("v_cache", C.POINTER(C.c_void_p)), ("max_seq", C.c_int32),
                ("token", C.c_void_p), ("token_log", C.c_void_p)]


class GncxLibraryMissing(RuntimeError):
    pass


_LIB = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load the built library and declare every signature.  Raises
    GncxLibraryMissing when it has not been built (there is no fallback)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise GncxLibraryMissing(f"{p} is not built: run __graft_entry__.build() or make -C {CSRC_DIR}")
    lib = C.CDLL(str(p), mode=C.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(lib: C.CDLL) -> None:
    """Raise if the last library call failed."""
    code = lib.gncx_hip_last_status()
    if code != 0:
        raise RuntimeError(f"gncx_llm_core error {code}: {lib.gncx_hip_last_error().decode()}")


def import_from(repo_root: str | os.PathLike):
    """Import <repo_root>/gnc-x_amd as the package ``gncx_amd``."""
    if "gncx_amd" in sys.modules:
        return sys.modules["gncx_amd"]
    root = pathlib.Path(repo_root) / "gnc-x_amd"
    spec = importlib.util.spec_from_file_location("gncx_amd", root / "__init__.py",
                                                  submodule_search_locations=[str(root)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["gncx_amd"] = mod
    spec.loader.exec_module(mod)
    return mod
