"""CPU checks of the drop-in boundary: the library loads and exports every symbol the header
declares, with no GPU needed (no compute calls)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "glm-ssd_amd", "libglmssd_hip.so")
HDRS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include"))) if h.endswith(".h")]


def header_symbols(only=None):
    text = "".join(open(h).read() for h in HDRS if only is None or h.endswith(only))
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(gs_\w+)\s*\(", text, re.M)))


def test_header_declares_reference_surface():
    syms = header_symbols()
    for s in ["gs_dequant_f32", "gs_dequant_f16", "gs_gemv", "gs_gemv_batched", "gs_moe_gateup", "gs_moe_down",
              "gs_gemm", "gs_gather_rows", "gs_scatter_add_rows", "gs_swiglu", "gs_axpy", "gs_malloc",
              "gs_event_elapsed_ms", "gs_error_string", "gs_device_info", "gs_quant_q8_1"]:
        assert s in syms, s


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build first: __graft_entry__.build()"
    lib = ctypes.CDLL(LIB)
    for s in header_symbols():
        assert hasattr(lib, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (gs_\w+)", out))
    assert set(header_symbols()) <= exported
    # nothing undeclared leaks out under the gs_ prefix
    assert exported - set(header_symbols()) == set()


def test_python_binding_covers_header():
    import glmssd
    from glmssd import gguf
    missing = [s for s in header_symbols("glmssd.h") if s not in glmssd.SIGNATURES and s != "gs_error_string"]
    assert not missing, missing
    missing = [s for s in header_symbols("glmssd_gguf.h") if s not in gguf._SIGS]
    assert not missing, missing


def test_moebatch_layout_matches_reference():
    import glmssd
    # crates/cuda/src/lib.rs:417-424: 3*16 pointers + 2*16 floats + int (+ tail padding)
    assert ctypes.sizeof(glmssd.MoeBatch) == 3 * 16 * 8 + 2 * 16 * 4 + 8
    assert glmssd.MoeBatch.n.offset == 3 * 16 * 8 + 2 * 16 * 4


def test_geometry_matches_oracle():
    import glmssd
    import oracle as O
    for ty in glmssd.TYPE_NAMES:
        assert glmssd.block(ty) == O.block(ty)
    assert glmssd.row_bytes(glmssd.GgmlType.IQ2_XXS, 1536) == 396
    with pytest.raises(ValueError):
        glmssd.row_bytes(glmssd.GgmlType.Q4_K, 100)


def test_kernels_embedded_for_gfx950():
    # each embedded code object is an AMDGPU ELF for gfx950; kernel names are present as text
    data = open(LIB, "rb").read()
    for name in [b"gs_k_stream_16_1_1", b"gs_k_stream_8_0_1", b"gs_k_dequant_f32_16", b"gs_k_quant_q8_1"]:
        assert name in data, name
    assert b"gfx950" in data


def test_expert_ptrs_layout():
    import glmssd
    assert ctypes.sizeof(glmssd.ExpertPtrs) == 24
    assert glmssd.ExpertPtrs.down.offset == 16


def test_group_pairs_matches_engine_grouping():
    from glmssd.moe import group_pairs
    import numpy as np
    rng = np.random.default_rng(0)
    routes = [[(int(e), float(rng.random())) for e in rng.choice(10, 3, replace=False)] for _ in range(7)]
    offs, idx, w, pe = group_pairs(routes, 10)
    assert offs[0] == 0 and offs[-1] == 21 and np.all(np.diff(offs) >= 0)
    # brute force: pairs of expert e are exactly the tokens routed to e, in token order
    for e in range(10):
        want = [(t, wt) for t, r in enumerate(routes) for (ee, wt) in r if ee == e]
        got = list(zip(idx[offs[e]:offs[e + 1]].tolist(), w[offs[e]:offs[e + 1]].tolist()))
        assert [g[0] for g in got] == [t for t, _ in want]
        assert np.allclose([g[1] for g in got], [wt for _, wt in want])
        assert np.all(pe[offs[e]:offs[e + 1]] == e)
    with pytest.raises(ValueError):
        group_pairs([[(10, 1.0)]], 10)
