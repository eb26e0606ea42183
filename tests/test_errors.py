"""Argument validation of the C ABI: bad arguments return hipErrorInvalidValue (1) without
launching, as the reference returns cudaErrorInvalidValue (quants.cu:225-241,380-397;
gemm.cu:110). These checks run before any device work, so they need no GPU."""
import ctypes as C

import glmssd as G

INVALID = 1
NULL = None


def test_gemv_rejects_bad_arguments():
    L = G.lib()
    assert L.gs_gemv(8, NULL, 34, 100, 4, NULL, 100, NULL, 4, 1, 0, NULL) == INVALID      # K % 32
    assert L.gs_gemv(12, NULL, 144, 128, 4, NULL, 128, NULL, 4, 1, 0, NULL) == INVALID    # K % QK (256)
    assert L.gs_gemv(8, NULL, 34, 64, 4, NULL, 64, NULL, 4, 0, 0, NULL) == INVALID        # B < 1
    assert L.gs_gemv(8, NULL, 34, 64, 4, NULL, 64, NULL, 4, 9, 0, NULL) == INVALID        # B > 8
    assert L.gs_gemv(99, NULL, 34, 64, 4, NULL, 64, NULL, 4, 1, 0, NULL) == INVALID       # unknown type
    assert L.gs_gemv(8, C.c_void_p(1), 34, 64, 4, NULL, 64, NULL, 4, 1, 0, NULL) == INVALID  # odd W


def test_dequant_rejects_bad_arguments():
    L = G.lib()
    assert L.gs_dequant_f32(8, NULL, 0, NULL, NULL) == INVALID
    assert L.gs_dequant_f32(8, NULL, 36, NULL, NULL) == INVALID     # not a whole block
    assert L.gs_dequant_f32(16, NULL, 32, NULL, NULL) == INVALID
    assert L.gs_dequant_f32(5, NULL, 32, NULL, NULL) == INVALID     # unknown type
    assert L.gs_quant_q8_1(NULL, NULL, 48, NULL) == INVALID


def test_moe_rejects_bad_batches():
    L = G.lib()
    b = G.MoeBatch()
    b.n = 0
    assert L.gs_moe_gateup(16, C.byref(b), 1, 1056, 4096, 1536, NULL, NULL, 0.0, NULL) == INVALID
    b.n = 17
    assert L.gs_moe_gateup(16, C.byref(b), 1, 1056, 4096, 1536, NULL, NULL, 0.0, NULL) == INVALID
    b.n = 8
    assert L.gs_moe_gateup(16, C.byref(b), 3, 1056, 4096, 1536, NULL, NULL, 0.0, NULL) == INVALID   # nt > 2
    assert L.gs_moe_down(16, C.byref(b), 0, 396, 1536, 4096, NULL, NULL, NULL) == INVALID
    assert L.gs_moe_down(16, C.byref(b), 1, 396, 1000, 4096, NULL, NULL, NULL) == INVALID          # K % 256


def test_gemm_rejects_bad_arguments():
    L = G.lib()
    assert L.gs_gemm(8, NULL, 34, 48, 4, NULL, 48, NULL, 4, 2, 0, 1, 0, 0, 0, NULL) == INVALID    # K % 32
    assert L.gs_gemm(8, NULL, 34, 64, 4, NULL, 64, NULL, 4, 0, 0, 1, 0, 0, 0, NULL) == INVALID    # N < 1
    assert L.gs_gemm(8, NULL, 34, 64, 4, NULL, 66, NULL, 4, 2, 0, 1, 0, 0, 0, NULL) == INVALID    # x_stride % 4


def test_zero_sized_row_ops_are_noops():
    L = G.lib()
    assert L.gs_gather_rows(NULL, NULL, NULL, 0, 16, NULL) == 0
    assert L.gs_scatter_add_rows(NULL, NULL, NULL, NULL, 0, 16, NULL) == 0
    assert L.gs_swiglu(NULL, NULL, NULL, 0, 0.0, NULL) == 0
    assert L.gs_axpy(NULL, NULL, 1.0, 0, NULL) == 0
