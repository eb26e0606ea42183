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


def test_moe_grouped_rejects_bad_arguments():
    L = G.lib()
    P = C.c_void_p
    x, y, tab, offs, idx, w, work = (P(256 * i) for i in range(1, 8))

    def call(ty=16, n_exp=288, n_pairs=64, n_tok=8, K=4096, n_ff=1536, rs_gu=1056, rs_dn=396, xx=x, wk=work,
             wb=1 << 30):
        return L.gs_moe_grouped(ty, ty, tab, n_exp, offs, idx, w, n_pairs, n_tok, rs_gu, K, n_ff, rs_dn, xx, y, 0.0,
                                wk, wb, NULL)
    assert call(ty=12) == INVALID                    # only IQ2_XXS
    assert call(n_exp=0) == INVALID
    assert call(n_exp=1025) == INVALID
    assert call(K=4000) == INVALID                   # not whole super-blocks
    assert call(n_ff=256, rs_dn=66) == INVALID       # fewer than two super-blocks per row
    assert call(rs_gu=1055) == INVALID               # odd row stride
    assert call(rs_gu=66) == INVALID                 # row stride shorter than a row
    assert call(xx=P(258)) == INVALID                # x not 16-byte aligned
    assert call(wk=P(300)) == INVALID                # workspace not 256-byte aligned
    assert call(wb=1024) == INVALID                  # workspace too small
    assert call(n_pairs=0) == 0                      # nothing to do, nothing launched
    n = C.c_size_t()
    assert L.gs_moe_grouped_workspace(512, 4096, 4096, 1536, C.byref(n)) == 0
    assert n.value >= 512 * 4096 * 2 + 4096 * 1536 * 6   # x16, h (f32) and h16
