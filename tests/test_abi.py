"""The C-ABI library on the CPU: it builds, loads, exports every entry point
include/gncx_llm_core.h declares with the reference's names, keeps the
reference's host-side bookkeeping (telemetry counters), and -- with no GPU --
fails loudly instead of computing on the CPU."""
from __future__ import annotations

import ctypes as C
import pathlib
import re
import subprocess

import numpy as np
import pytest

import synth
from conftest import ROOT, gncx, ptr

HEADER = ROOT / "include" / "gncx_llm_core.h"
REF_CPP_EXPORTS = [  # the 48 names csrc/gncx_llm_kernels.cpp exports, in its order
    "gncx_gla_map_readonly", "gncx_gla_get_base_ptr", "gncx_gla_unmap", "gncx_ram_alloc_colored", "gncx_ram_alloc",
    "gncx_ram_get_ptr", "gncx_ram_get_ddr3_bank", "gncx_ram_get_l1_set", "gncx_ram_free", "gncx_ram_copy_chunk",
    "gncx_gla_prefetch_range", "gncx_genome_get_layer_coordinate", "gncx_fetch_token_embedding_q8_0",
    "gncx_fetch_token_embedding_q6_k", "gncx_fetch_token_embedding_bf16", "gncx_rmsnorm_and_encode_4phase",
    "gncx_rmsnorm_inplace_heads", "gncx_xfold_universal_matvec", "gncx_xfold_q4_0_matvec",
    "gncx_xfold_universal_matbatch", "gncx_xfold_q4_0_matbatch", "gncx_universal_lm_head_logits",
    "gncx_q8_0_lm_head_logits", "gncx_apply_rope_xor11_ext", "gncx_apply_rope_xor11", "gncx_mqa_attention_step_ext",
    "gncx_mqa_attention_step", "gncx_geglu_activation", "gncx_swiglu_activation", "gncx_geo_mm_create",
    "gncx_geo_mm_destroy", "gncx_geo_alloc", "gncx_geo_free", "gncx_geo_fragmentation", "gncx_geo_used",
    "gncx_geo_capacity", "gncx_lora_init_adapter", "gncx_lora_forward_add", "gncx_lora_backward_step",
    "gncx_mezo_perturb_params", "gncx_mezo_update_params", "gncx_cross_entropy_loss", "gncx_project_layer_3d_point",
    "gncx_cosine_similarity", "gncx_vector_l2_normalize", "gncx_mean_pooling", "gncx_bidirectional_attention_gqa",
    "gncx_bidirectional_attention",
]


def header_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(gncx_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def built():
    if not gncx.LIB_PATH.exists():
        out = subprocess.run(["make", "-C", str(gncx.CSRC_DIR), "-j8"], capture_output=True, text=True)
        assert out.returncode == 0, out.stdout + out.stderr
    return gncx.LIB_PATH


def exported(path: pathlib.Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True)
    return {ln.split()[-1] for ln in out.stdout.splitlines() if " T " in ln}


def test_header_declares_reference_names():
    fns = header_functions()
    for name in REF_CPP_EXPORTS:
        assert name in fns, name


def test_library_exports_every_declared_symbol(built):
    syms = exported(built)
    missing = [f for f in header_functions() if f not in syms]
    assert not missing, missing
    # nothing else leaks out of the library
    assert all(s.startswith("gncx_") for s in syms), sorted(s for s in syms if not s.startswith("gncx_"))


def test_ctypes_signatures_cover_header(built):
    assert set(header_functions()) == set(gncx.SIGNATURES)
    lib = gncx.load()
    for name in gncx.SIGNATURES:
        assert getattr(lib, name) is not None


def test_exports_match_reference_signatures(built, ref):
    """The reference build exports exactly these 48 names, and so does ours."""
    ref_syms = exported(pathlib.Path(ref.lib._name))
    assert len(REF_CPP_EXPORTS) == 48
    assert ref_syms == set(REF_CPP_EXPORTS), sorted(ref_syms ^ set(REF_CPP_EXPORTS))
    assert set(REF_CPP_EXPORTS) <= exported(built)


# ---- prototypes: return type and parameter types, in order ---------------
REF_CPP = pathlib.Path("/root/reference/csrc/gncx_llm_kernels.cpp")
REF_CDEF = pathlib.Path("/root/reference/lua/gncx_streamer.lua")


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return re.sub(r"--[^\n]*", " ", text) if "ffi.cdef" in text else text


def _norm_type(t: str) -> str:
    t = re.sub(r"\b(__restrict__|__restrict|restrict|extern|GNCX_LLM_API|GNCX_API)\b", " ", t)
    t = t.replace('"C"', " ")
    t = re.sub(r"\bstruct\s+", "", t)
    t = re.sub(r"\b(GNCX\w+?)Struct\b", r"\1", t)  # the LuaJIT cdef's typedef names
    t = re.sub(r"\s*\*\s*", "*", t)
    return re.sub(r"\s+", " ", t).strip()


def _param_type(p: str) -> str | None:
    p = p.strip()
    if p in ("", "void"):
        return None
    m = re.match(r"^(.*[\s*])([A-Za-z_]\w*)$", p)  # the type, then the parameter's name
    return _norm_type(m.group(1) if m else p)


def prototypes(text: str, prefix: str = "") -> dict[str, tuple[str, tuple[str, ...]]]:
    """name -> (return type, parameter types) of every gncx_* prototype or
    definition in C text; with prefix, only those whose declaration starts
    with it (e.g. the export macro)."""
    text = _strip_comments(text)
    text = re.sub(r"^[ \t]*#[^\n]*", " ", text, flags=re.M)  # preprocessor lines
    out = {}
    for m in re.finditer(r"\b(gncx_\w+)\s*\(", text):
        name = m.group(1)
        # the declaration starts after the previous statement or block end
        start = max(text.rfind(c, 0, m.start()) for c in ";{}]")
        head = text[start + 1:m.start()]
        if (prefix and prefix not in head) or "(" in head or "=" in head or "return" in head.split():
            continue
        depth, i = 1, m.end()
        while depth and i < len(text):
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        if not text[i:].lstrip().startswith((";", "{")):
            continue  # a call, not a declaration
        params = text[m.end():i - 1]
        out[name] = (_norm_type(head), tuple(t for t in (_param_type(p) for p in params.split(",")) if t is not None))
    return out


def test_header_prototypes_parse():
    ours = prototypes(HEADER.read_text())
    assert set(REF_CPP_EXPORTS) <= set(ours)
    assert ours["gncx_xfold_universal_matvec"] == (
        "void", ("const uint8_t*", "size_t", "int32_t", "const float*", "const GNCXCompactToken*", "int32_t",
                 "int32_t", "float*", "GNCXTelemetryStats*"))


@pytest.mark.skipif(not (REF_CPP.exists() and REF_CDEF.exists()), reason="reference sources absent")
def test_prototypes_match_reference_definitions_and_ffi_cdef():
    """Every one of the 48 reference entry points: the same return type and
    the same parameter types in the same order in include/gncx_llm_core.h,
    in the reference's GNCX_LLM_API definitions (csrc/gncx_llm_kernels.cpp)
    and in the LuaJIT cdef that binds them (lua/gncx_streamer.lua:16-252)."""
    ours = prototypes(HEADER.read_text())
    ref = prototypes(REF_CPP.read_text(), prefix="GNCX_LLM_API")
    lua = REF_CDEF.read_text()
    cdef = prototypes(lua[lua.index("ffi.cdef[["):lua.index("]]", lua.index("ffi.cdef[["))])
    assert set(ref) == set(REF_CPP_EXPORTS), sorted(set(ref) ^ set(REF_CPP_EXPORTS))
    for name in REF_CPP_EXPORTS:
        assert ours[name] == ref[name], (name, ours[name], ref[name])
        if name in cdef:  # the streamer binds a subset (lua/gncx_streamer.lua:16-252)
            assert ours[name] == cdef[name], (name, ours[name], cdef[name])
    assert len(set(cdef) & set(REF_CPP_EXPORTS)) >= 40


def _has_gpu(lib) -> bool:
    n = C.c_int(0)
    try:
        hip = C.CDLL("libamdhip64.so")
    except OSError:
        return False
    return hip.hipGetDeviceCount(C.byref(n)) == 0 and n.value > 0


def test_no_gpu_means_loud_failure_not_cpu_fallback(built):
    lib = gncx.load()
    if _has_gpu(lib):
        pytest.skip("a GPU is visible; the no-device path is exercised on CPU-only hosts")
    k, n = 256, 8
    w = synth.make_weights(12, n, k, seed=1)
    x = synth.make_activations(1, k, seed=2)
    y = np.full(n, 7.0, dtype=np.float32)
    lib.gncx_xfold_universal_matvec(ptr(w), 0, 12, ptr(x), None, k, n, ptr(y), None)
    assert lib.gncx_hip_last_status() != 0
    assert np.all(y == 7.0), "output must be left untouched when there is no device"


def test_telemetry_matches_reference(built, ref):
    """Counters follow cpp:1464-1470 and cpp:1686-1691 exactly, with or
    without a device (they are host bookkeeping)."""
    lib = gncx.load()
    k, n, b = 512, 16, 3
    w = synth.make_weights(14, n, k, seed=3)
    x = synth.make_activations(1, k, seed=4)
    xb = synth.make_activations(b, k, seed=5)
    y = np.zeros(n, np.float32)
    yb = np.zeros((b, n), np.float32)
    tokens = (gncx.GNCXCompactToken * k)()
    rng = np.random.default_rng(6)
    for i in range(k):
        tokens[i].phase_2bit = int(rng.integers(0, 4))
        tokens[i].diag_d = int(rng.integers(0, 10))
    mine, theirs = gncx.GNCXTelemetryStats(), gncx.GNCXTelemetryStats()
    for L, t in ((lib, mine), (ref.lib, theirs)):
        L.gncx_xfold_universal_matvec(ptr(w), 0, 14, ptr(x), C.addressof(tokens), k, n, ptr(y), C.addressof(t))
        L.gncx_xfold_universal_matbatch(ptr(w), 0, 14, ptr(xb), b, k, n, ptr(yb), C.addressof(t))
    lib.gncx_hip_last_status()
    for f, _ in gncx.GNCXTelemetryStats._fields_:
        assert getattr(mine, f) == getattr(theirs, f), f
    assert mine.zero_origin_cancellations > 0


def test_decode_structs_match_header(tmp_path):
    """The ctypes mirrors of the native decode step's structs have the C
    layout the header declares (sizes and every field offset, from a program
    compiled against include/gncx_llm_core.h)."""
    fields = {
        "GNCXDecodeTensor": ("offset", "ggml_type"),
        "GNCXDecodeLayer": ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_q_norm", "attn_k_norm", "attn_output",
                            "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"),
        "GNCXDecodeModel": ("base", "layers", "token_embd", "output_norm", "n_layers", "embed", "n_heads",
                            "n_kv_heads", "head_dim", "ffn", "vocab", "qk_norm", "eps", "rope_base", "attn_scale"),
        "GNCXDecodeState": ("hidden", "q", "k", "v", "attn", "proj", "normed", "gate", "up", "act", "logits",
                            "k_cache", "v_cache", "max_seq", "token", "token_log"),
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "gncx_llm_core.h"', "int main(void) {"]
    for s, fs in fields.items():
        lines.append(f'printf("{s} sizeof %zu\\n", sizeof({s}));')
        for f in fs:
            lines.append(f'printf("{s} {f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for ln in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        s, f, v = ln.split()
        got[(s, f)] = int(v)
    py = {"GNCXDecodeTensor": gncx.DecodeTensor, "GNCXDecodeLayer": gncx.DecodeLayer,
          "GNCXDecodeModel": gncx.DecodeModel, "GNCXDecodeState": gncx.DecodeState}
    for s, fs in fields.items():
        assert C.sizeof(py[s]) == got[(s, "sizeof")], s
        for f in fs:
            assert getattr(py[s], f).offset == got[(s, f)], (s, f)


def test_streamer_replay_library_links_against_the_core(built):
    """gncx_streamer_replay.so (the native caller used to time the unchanged
    streamer's call sequence) loads, resolves its calls in this very core
    library, and exports its one entry point."""
    replay = gncx.LIB_PATH.parent / "gncx_streamer_replay.so"
    assert replay.exists()
    lib = gncx.load()
    so = C.CDLL(str(replay))
    assert so.gncx_replay_forward_token is not None
    out = subprocess.run(["readelf", "-d", str(replay)], capture_output=True, text=True, check=True).stdout
    assert "gncx_llm_core.so" in out
    # its NEEDED entry binds to the core by SONAME (the reference build, loaded
    # by path in the same process, has none), so the library state is shared
    core = subprocess.run(["readelf", "-d", str(gncx.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert "Library soname: [gncx_llm_core.so]" in core
    maps = pathlib.Path(f"/proc/{__import__('os').getpid()}/maps").read_text()
    ours = {ln.split()[-1] for ln in maps.splitlines() if ln.endswith("gnc-x_amd/bin/gncx_llm_core.so")}
    assert len(ours) == 1, ours
    assert lib.gncx_hip_last_status is not None
