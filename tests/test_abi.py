"""The C-ABI library loads and exports exactly what include/gpic_fp8.h declares; argument validation returns the
documented status codes before anything is launched (no GPU needed)."""
import ctypes
import os
import re

import pytest

from gpic_fp8 import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gpic_fp8.h")


def declared():
    src = open(HEADER).read()
    return set(re.findall(r"^(?:int|void|size_t|const char \*)\s*(gpic_fp8_\w+)\(", src, flags=re.M))


def test_header_declares_the_bound_functions():
    assert declared() == set(L.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.gpic_fp8_version().startswith(b"gpic_fp8")


def test_status_strings():
    lib = L.lib()
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.gpic_fp8_status_string(code)
    assert lib.gpic_fp8_status_string(-99) == b"unknown status"


def test_cast_workspace_size():
    assert L.lib().gpic_fp8_cast_workspace_bytes() >= 4096


def test_validation_codes():
    lib = L.lib()
    ws = ctypes.create_string_buffer(4096 + 16)
    wsp = (ctypes.addressof(ws) + 15) // 16 * 16
    # negative size / null output
    assert lib.gpic_fp8_tcast(None, 0, -1, None, wsp, wsp, None) == -1
    assert lib.gpic_fp8_tcast(None, 0, 0, None, None, wsp, None) == -1
    # unsupported dtype
    assert lib.gpic_fp8_tcast(wsp, 7, 16, wsp, wsp, wsp, None) == -2
    # misaligned input
    assert lib.gpic_fp8_tcast(wsp + 2, 0, 16, wsp, wsp, wsp, None) == -4
    # the allocation-free cast checks the same arguments before it sets anything up
    na = lib.gpic_fp8_tcast_noalloc
    assert na(None, 0, -1, None, wsp, None) == -1
    assert na(wsp, 0, 16, wsp, None, None) == -1
    assert na(wsp, 7, 16, wsp, wsp, None) == -2
    assert na(wsp + 2, 0, 16, wsp, wsp, None) == -4
    # transposing cast: columns must be a multiple of 16, ldt >= rows
    assert lib.gpic_fp8_tcast_t(wsp, 0, 4, 24, wsp, wsp, 16, wsp, wsp, None) == -3
    # grouped transposing casts: a negative count or null arrays; each tensor checked as gpic_fp8_tcast_t checks it
    tg = lib.gpic_fp8_tcast_t_group
    assert tg(-1, None, 0, None, None, None, None, None, None, wsp, None) == -1
    assert tg(1, None, 0, None, None, None, None, None, None, wsp, None) == -1
    assert tg(0, None, 0, None, None, None, None, None, None, wsp, None) == 0
    P = lambda *v: (ctypes.c_void_p * len(v))(*v)
    I = lambda *v: (ctypes.c_int64 * len(v))(*v)
    good = (P(wsp, wsp), 0, I(4, 4), I(16, 16), P(wsp, wsp), P(wsp, wsp), I(16, 16), P(wsp, wsp), wsp, None)
    assert tg(2, good[0], 7, *good[2:]) == -2                                    # unsupported dtype
    assert tg(2, good[0], 0, I(4, 4), I(16, 24), *good[4:]) == -3                # the second tensor's columns
    assert tg(2, good[0], 0, I(4, 20), I(16, 16), good[4], good[5], I(16, 16), *good[7:]) == -3   # ldt < rows
    assert tg(2, P(wsp, wsp + 2), 0, *good[2:]) == -4                           # misaligned second source
    assert lib.gpic_fp8_tcast_t(wsp, 0, 40, 32, wsp, wsp, 32, wsp, wsp, None) == -3
    # the attention output's head-merging cast: extents and strides >= 0, D % 16, strides % 8, 16-byte pointers,
    # word indices below 2^31
    th = lib.gpic_fp8_tcast_heads
    assert th(wsp, -1, 2, 4, 16, 128, 64, 16, wsp, wsp, wsp, None) == -1
    assert th(wsp, 1, 2, 4, 16, 128, -64, 16, wsp, wsp, wsp, None) == -1
    assert th(wsp, 1, 2, 4, 16, 128, 64, 16, wsp, None, wsp, None) == -1
    assert th(None, 1, 2, 4, 16, 128, 64, 16, wsp, wsp, wsp, None) == -1
    assert th(wsp, 1, 2, 4, 24, 192, 96, 24, wsp, wsp, wsp, None) == -3
    assert th(wsp, 1, 2, 4, 16, 128, 68, 16, wsp, wsp, wsp, None) == -4
    assert th(wsp + 8, 1, 2, 4, 16, 128, 64, 16, wsp, wsp, wsp, None) == -4
    assert th(wsp, 1, 2, 4, 16, 128, 64, 16, wsp + 8, wsp, wsp, None) == -4
    assert th(wsp, 2, 2, 4, 16, 1 << 34, 64, 16, wsp, wsp, wsp, None) == -3
    assert th(wsp, 1 << 20, 16, 1024, 64, 1 << 20, 64, 1024, wsp, wsp, wsp, None) == -3
    # SwiGLU: H % 8, strides
    assert lib.gpic_fp8_swiglu_tcast(wsp, 4, 12, 24, wsp, 12, wsp, wsp, None) == -3
    assert lib.gpic_fp8_swiglu_tcast(wsp, 4, 16, 16, wsp, 16, wsp, wsp, None) == -3
    assert lib.gpic_fp8_swiglu_bwd(wsp, wsp, 4, 16, 32, 8, wsp, wsp, wsp, wsp, None) == -3
    assert lib.gpic_fp8_swiglu_tcast_t(wsp, 40, 16, 32, None, wsp, 16, wsp, 32, wsp, wsp, None) == -3
    # product cast with qt = NULL (q only): ldt must be 0; H % 8 suffices there, H % 16 with qt
    assert lib.gpic_fp8_swiglu_tcast_t(wsp, 4, 16, 32, None, wsp, 16, None, 16, wsp, wsp, None) == -1
    assert lib.gpic_fp8_swiglu_tcast_t(wsp, 4, 24, 48, None, wsp, 24, wsp, 16, wsp, wsp, None) == -3
    assert lib.gpic_fp8_swiglu_tcast_t(wsp, 4, 12, 24, None, wsp, 16, None, 0, wsp, wsp, None) == -3
    # SwiGLU backward without dz: needs the transposed output (dzqt, ldt > 0); a given dz must be aligned
    b = lib.gpic_fp8_swiglu_bwd_t
    assert b(wsp, wsp, 4, 16, 32, 16, None, wsp, wsp, 0, wsp, wsp, None) == -1
    assert b(wsp, wsp, 4, 16, 32, 16, None, wsp, None, 16, wsp, wsp, None) == -1
    assert b(wsp, wsp, 4, 16, 32, 16, wsp + 8, wsp, wsp, 16, wsp, wsp, None) == -4
    # the norm sites' producer: C % 4, rows % ntok, strides, nothing to write, misaligned weight
    nm = lib.gpic_fp8_res_mod_rmsnorm
    assert nm(wsp, None, None, 0, wsp, wsp, 256, wsp, 256, 4, 2, 130, 1e-6, None, None, wsp, wsp, wsp, wsp, None) == -3
    assert nm(wsp, None, None, 0, wsp, wsp, 256, wsp, 256, 5, 2, 256, 1e-6, None, None, wsp, wsp, wsp, wsp, None) == -3
    assert nm(wsp, None, None, 0, wsp, wsp, 255, wsp, 256, 4, 2, 256, 1e-6, None, None, wsp, wsp, wsp, wsp, None) == -3
    assert nm(wsp, None, None, 0, wsp, wsp, 256, wsp, 256, 4, 2, 256, 1e-6, None, None, wsp, None, None, wsp, None) == -1
    assert nm(wsp, None, None, 0, wsp, wsp, 256, wsp, 256, 4, 2, 256, 1e-6, None, None, wsp, None, wsp, wsp, None) == -1
    assert nm(wsp, None, None, 0, wsp + 8, wsp, 256, wsp, 256, 4, 2, 256, 1e-6, None, None, wsp, wsp, wsp, wsp,
              None) == -4
    assert nm(wsp, wsp, None, 256, wsp, wsp, 256, wsp, 256, 4, 2, 256, 1e-6, wsp, None, wsp, wsp, wsp, wsp, None) == -1
    # the norm's backward: C % 4 and <= 2048, rows % ntok, site-1 arguments, workspace size, alignment
    nb = lib.gpic_fp8_res_mod_rmsnorm_bwd
    nbw = lib.gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes
    assert nbw(4, 2, 256) == 4 * 2 * 256 * 4 and nbw(4, 3, 256) == 0 and nbw(0, 1, 256) == 0
    assert nb(wsp, None, wsp, None, None, 0, wsp, wsp, 256, wsp, 4, 2, 130, wsp, None, wsp, wsp, None, wsp, wsp, 1 << 20,
              None) == -3
    assert nb(wsp, None, wsp, None, None, 0, wsp, wsp, 4096, wsp, 4, 2, 4096, wsp, None, wsp, wsp, None, wsp, wsp,
              1 << 20, None) == -3
    assert nb(wsp, None, wsp, None, None, 0, wsp, wsp, 256, wsp, 5, 2, 256, wsp, None, wsp, wsp, None, wsp, wsp, 1 << 20,
              None) == -3
    assert nb(wsp, wsp, wsp, None, None, 0, wsp, wsp, 256, wsp, 4, 2, 256, wsp, None, wsp, wsp, None, wsp, wsp, 1 << 20,
              None) == -1
    assert nb(wsp, None, wsp, wsp, None, 256, wsp, wsp, 256, wsp, 4, 2, 256, wsp, wsp, wsp, wsp, wsp, wsp, wsp, 1 << 20,
              None) == -1
    assert nb(wsp, None, wsp, None, None, 0, wsp, wsp, 256, wsp, 4, 2, 256, wsp, None, wsp, wsp, None, wsp, wsp, 16,
              None) == -5
    assert nb(wsp + 8, None, wsp, None, None, 0, wsp, wsp, 256, wsp, 4, 2, 256, wsp, None, wsp, wsp, None, wsp, wsp,
              1 << 20, None) == -4
    # GEMM: K % 16, N % 16, leading dimensions, null scales
    g = lib.gpic_fp8_gemm
    assert g(wsp, 24, wsp, wsp, 24, wsp, None, wsp, 16, 4, 16, 24, 1, None, 0, None) == -3
    assert g(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 24, 4, 24, 32, 1, None, 0, None) == -3
    assert g(wsp, 16, wsp, wsp, 32, wsp, None, wsp, 16, 4, 16, 32, 1, None, 0, None) == -3
    assert g(wsp, 32, None, wsp, 32, wsp, None, wsp, 16, 4, 16, 32, 1, None, 0, None) == -1
    # the epilogue's C offsets are 32-bit: ldc < 2^22 (a larger one would wrap them)
    assert g(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 1 << 22, 4, 16, 32, 1, None, 0, None) == -3
    assert g(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 1 << 30, 4, 16, 32, 1, None, 0, None) == -3
    # empty output: nothing to do
    assert g(None, 32, wsp, None, 32, wsp, None, None, 16, 0, 16, 32, 1, None, 0, None) == 0
    # MN-major GEMM: M % 16, N % 16, lda >= M, ldb >= N, K * ld < 2^31, null scales, misaligned operand
    mn = lib.gpic_fp8_gemm_mn
    assert mn(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 32, 24, 32, 5, None, 0, None) == -3
    assert mn(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 32, 32, 24, 5, None, 0, None) == -3
    assert mn(wsp, 16, wsp, wsp, 32, wsp, None, wsp, 32, 32, 32, 5, None, 0, None) == -3
    assert mn(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 32, 32, 32, 1 << 27, None, 0, None) == -3
    assert mn(wsp, 32, None, wsp, 32, wsp, None, wsp, 32, 32, 32, 5, None, 0, None) == -1
    assert mn(wsp + 8, 32, wsp, wsp, 32, wsp, None, wsp, 32, 32, 32, 5, None, 0, None) == -4
    assert mn(None, 32, wsp, None, 32, wsp, None, None, 32, 0, 32, 5, None, 0, None) == 0
    assert mn(wsp, 32, wsp, wsp, 32, wsp, None, wsp, 1 << 22, 32, 32, 5, None, 0, None) == -3


def test_single_pass_knob_is_host_only():
    """gpic_fp8_set_single_pass only records the setting (no device call): safe without a GPU; defaults restored."""
    L.set_single_pass(False, 0)
    L.set_single_pass(True, -1)


def test_loader_fails_loudly_without_library(monkeypatch, tmp_path):
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        L.lib()
