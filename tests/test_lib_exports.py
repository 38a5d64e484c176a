"""The C ABI library on CPU: it loads, exports every symbol include/loopback_read.h declares, and its host-side
argument checks reject bad calls before any launch (no GPU is touched by these calls)."""
import ctypes
import os
import re

import pytest

from loopback_amd import build as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "loopback_read.h")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ldr_\w+)\s*\(", txt)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(B.LIB):
        B.build(verbose=False)
    from loopback_amd import _lib
    return _lib


def test_header_declares_entry_points():
    names = declared()
    assert "ldr_read_fwd" in names and "ldr_read_bwd1" in names and "ldr_dv_assemble" in names
    assert len(names) >= 13


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(lib.PATH)
    missing = [n for n in declared() if not hasattr(raw, n)]
    assert not missing, missing
    assert set(declared()) == set(lib.SIGNATURES), "the ctypes signature table must cover the header exactly"


def test_abi_version_and_messages(lib):
    with open(HEADER) as f:
        header = int(re.search(r"#define LDR_ABI_VERSION (\d+)", f.read()).group(1))
    assert lib.LIB.ldr_abi_version() == lib.ABI_VERSION == header
    for code in (0, -1, -2, -3, -4):
        assert lib.LIB.ldr_strerror(code).decode()


@pytest.mark.parametrize("d,expect", [(2048, (4, 64)), (768, (3, 32)), (1024, (2, 64)), (64, (1, 8)),
                                      (1536, (3, 64)), (3072, (3, 128)), (256, (1, 32)), (8192, (4, 256))])
def test_row_layout(lib, d, expect):
    vpt, tpr = lib.row_layout(d)
    assert (vpt, tpr) == expect
    assert vpt * tpr * 8 >= d and tpr & (tpr - 1) == 0


@pytest.mark.parametrize("d", [0, 7, 100, 8200])
def test_row_layout_rejects(lib, d):
    with pytest.raises(RuntimeError):
        lib.row_layout(d)


def test_bwd1_parts(lib):
    assert lib.bwd1_parts(16384, 2048) == 512
    assert lib.bwd1_parts(20, 2048) == 1          # 32-token tiles
    assert lib.bwd1_parts(65, 2048) == 3
    assert lib.bwd1_parts(0, 2048) == 0


def test_argument_checks_before_launch(lib):
    L = lib.LIB
    null = ctypes.c_void_p(0)
    assert L.ldr_rstd_fwd(null, null, 16, 64, 1e-6, 1, null) == -1
    assert L.ldr_rstd_fwd(ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 0, 1e-6, 1, null) == -1
    assert L.ldr_rstd_bwd(ctypes.c_void_p(4096), ctypes.c_void_p(4096), ctypes.c_void_p(4096), ctypes.c_void_p(4096),
                          16, -8, 1, null) == -1
    # (the scale takes any width and alignment; the read's vector kernels do not)
    one_v = lib.u64_array([4096])
    assert L.ldr_dots_online(one_v, 1, ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 16, 60, 1, null) == -2
    assert L.ldr_dots_online(lib.u64_array([4100]), 1, ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 16, 64, 1,
                             null) == -3
    assert L.ldr_rstd_fwd(ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 64, 1e-6, 7, null) == -4
    # fp16 (code 2) is an update dtype of every entry point (no tokens: nothing launched); code 3 is none
    assert L.ldr_rstd_fwd(null, null, 0, 64, 1e-6, lib.F16, null) == 0
    assert L.ldr_dots_online(one_v, 1, ctypes.c_void_p(4096), null, 0, 0, 64, lib.F16, null) == 0
    assert L.ldr_dots_online(one_v, 1, ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 16, 64, 3, null) == -4
    assert L.ldr_write_dots(null, null, null, null, null, null, 4, 4, null, 0, 64, 0, 1e-6, lib.F16, null) == 0
    too_many = lib.u64_array([4096] * 65)
    assert L.ldr_dots_online(too_many, 65, ctypes.c_void_p(4096), ctypes.c_void_p(4096), 16, 16, 64, 1, null) == -1
    p4 = ctypes.c_void_p(4096)
    # more queries than a stack holds; a first scored query past the last
    assert L.ldr_write_dots(p4, p4, p4, p4, p4, p4, 65, 0, p4, 16, 64, 16, 1e-6, 1, null) == -2
    assert L.ldr_write_dots(p4, p4, p4, p4, p4, p4, 4, 5, p4, 16, 64, 16, 1e-6, 1, null) == -1
    # scores of every dtype need the queries' operand table (the fp32 queries alone do not do)
    assert L.ldr_write_dots(p4, p4, p4, p4, p4, null, 4, 0, p4, 16, 64, 16, 1e-6, 1, null) == -1
    assert L.ldr_write_dots(p4, p4, p4, p4, p4, null, 4, 0, p4, 16, 64, 16, 1e-6, 0, null) == -1
    # no scores (j_lo == nq): neither is needed
    assert L.ldr_write_dots(null, null, null, null, null, null, 4, 4, null, 0, 64, 0, 1e-6, 1, null) == 0
    assert L.ldr_split_queries(null, 8, 64, p4, null) == -1
    assert L.ldr_split_queries(p4, 65, 64, p4, null) == -2
    assert L.ldr_split_queries(p4, 8, 64, ctypes.c_void_p(4100), null) == -3
    # the operand table's size: 64-column chunks x 16-query blocks x 3 parts x 2 halves x 64 lanes x 8 values
    assert L.ldr_query_parts_elems(31, 2048) == 32 * 2 * 3 * 2 * 64 * 8
    assert L.ldr_query_parts_elems(1, 8) == 3 * 2 * 64 * 8 and L.ldr_query_parts_elems(65, 64) == 0
    assert L.ldr_dv_assemble(too_many, too_many, too_many, 65, ctypes.c_void_p(4096), ctypes.c_void_p(4096), null,
                             null, 0.0, 0, ctypes.c_void_p(4096), null, 16, 64, 1, null) == -2
    # a misaligned added gradient
    assert L.ldr_dv_assemble(one_src := lib.u64_array([4096]), one_src, one_src, 1, ctypes.c_void_p(4096),
                             ctypes.c_void_p(4096), null, ctypes.c_void_p(4100), 0.0, 0, ctypes.c_void_p(4096), null,
                             16, 64, 1, null) == -3
    # a misaligned blend-gradient output
    one = lib.u64_array([4096])
    p = ctypes.c_void_p(4096)
    assert L.ldr_read_bwd1(one, one, 1, p, null, p, p, 16, p, p, 1, p, 1, 1.0, 0.125, p, 1, one, 0, p, 16, p, 64,
                           ctypes.c_void_p(4104), null, 0.5, 16, 64, 1, null) == -3
    assert L.ldr_blend_sum(too_many, 65, 0.5, 0, p, 16, 64, 1, null) == -2
    assert L.ldr_blend_sum(one, 1, 0.5, 0, ctypes.c_void_p(4100), 16, 64, 1, null) == -3
    assert L.ldr_blend_sum(one, 1, 0.5, 2, p, 16, 64, 1, null) == -1
    # the raw scores' row stride covers the tokens
    assert L.ldr_read_bwd1(one, one, 1, p, null, p, p, 8, p, p, 1, p, 1, 1.0, 0.125, p, 1, one, 0, p, 16, p, 64,
                           null, null, 0.0, 16, 64, 1, null) == -1
    # ... and the dq partials' row stride covers a row
    assert L.ldr_read_bwd1(one, one, 1, p, null, p, p, 16, p, p, 1, p, 1, 1.0, 0.125, p, 1, one, 0, p, 16, p, 56,
                           null, null, 0.0, 16, 64, 1, null) == -1
    # coefficient columns: n (as the read takes them) or n - 1 (fused bookkeeping), nothing else
    two = lib.u64_array([4096, 4096])
    assert L.ldr_read_fwd(two, two, 2, p, 16, p, null, 0.0, p, 3, p, 2, 1.0, 0.125, p, p, p, null, 16, 64, 1,
                          null) == -1
    # the one-pass online read needs the query and the score output (the backward's raw scores), both aligned
    assert L.ldr_read_fwd_online(two, two, 2, null, p, 16, p, null, 0.0, p, 2, p, 2, 1.0, 0.125, p, p, p, null, 16,
                                 64, 1, null) == -1
    assert L.ldr_read_fwd_online(two, two, 2, p, null, 16, p, null, 0.0, p, 2, p, 2, 1.0, 0.125, p, p, p, null, 16,
                                 64, 1, null) == -1
    assert L.ldr_read_fwd_online(two, two, 2, ctypes.c_void_p(4100), p, 16, p, null, 0.0, p, 2, p, 2, 1.0, 0.125, p,
                                 p, p, null, 16, 64, 1, null) == -3
    for width in (2048, 8192):   # one pass (rows in one wave) and two (wider rows)
        assert L.ldr_read_fwd_online(two, two, 2, p, p, 16, p, null, 0.0, p, 2, p, 2, 1.0, 0.01, p, p, p, null, 0,
                                     width, 1, null) == 0
    # the widest row (8192) is a shape every stacked entry point takes (no tokens: checked, nothing launched)
    assert L.ldr_dv_assemble(one_src, one_src, one_src, 1, p, p, null, null, 0.0, 0, p, null, 0, 8192, 1, null) == 0
    assert L.ldr_dv_assemble(one_src, one_src, one_src, 1, p, p, null, null, 0.0, 1, p, null, 0, 8192, 1, null) == 0
    assert L.ldr_dv_assemble(one_src, one_src, one_src, 1, p, p, null, null, 0.0, 2, p, null, 0, 8192, 1, null) == -1
    assert L.ldr_blend_sum(one, 1, 0.5, 0, p, 0, 8192, 1, null) == 0
    assert L.ldr_read_fwd(two, two, 2, p, 16, p, null, 0.0, p, 2, p, 2, 1.0, 0.01, p, p, p, null, 0, 8192, 1,
                          null) == 0
    assert L.ldr_read_bwd1(one, one, 1, p, null, p, p, 16, p, p, 1, p, 1, 1.0, 0.01, p, 1, one, 0, p, 16, p, 8192,
                           null, null, 0.0, 0, 8192, 1, null) == 0
    # zero tokens: accepted, nothing launched
    assert L.ldr_rstd_fwd(ctypes.c_void_p(4096), ctypes.c_void_p(4096), 0, 64, 1e-6, 1, null) == 0
    # ... also with the token-sized buffers NULL, as torch's empty tensors give them (never with tokens)
    nulls = lib.u64_array([0, 0])
    assert L.ldr_rstd_fwd(null, null, 0, 64, 1e-6, 1, null) == 0
    assert L.ldr_rstd_fwd(null, null, 1, 64, 1e-6, 1, null) == -1
    assert L.ldr_read_fwd(nulls, nulls, 2, null, 0, null, null, 0.0, null, 2, p, 2, 1.0, 0.125, null, null, null,
                          null, 0, 64, 1, null) == 0
    assert L.ldr_read_fwd(nulls, nulls, 2, null, 0, null, null, 0.0, null, 2, p, 2, 1.0, 0.125, null, null, null,
                          null, 1, 64, 1, null) == -1
    assert L.ldr_dv_assemble(lib.u64_array([0]), lib.u64_array([0]), one, 1, null, null, null, null, 0.0, 0, null,
                             null, 0, 64, 1, null) == 0
    assert L.ldr_read_bwd1(nulls, nulls, 2, null, null, null, null, 0, null, null, 2, p, 2, 1.0, 0.125, null, 2,
                           nulls, 0, null, 0, p, 64, null, null, 0.0, 0, 64, 1, null) == 0


def test_any_shape_argument_checks_before_launch(lib):
    """The any-shape entry points take any width >= 1 and up to LDR_ANY_MAX_SOURCES sources at element alignment,
    and refuse the rest before any launch (their device address arrays are not read on the host)."""
    L = lib.LIB
    null = None
    p = 4096                         # a stand-in address: every call below is refused or has no tokens
    odd = 4097                       # not element-aligned for bf16
    many = lib.ANY_MAX_SOURCES + 1
    rd = lambda n, d, base=p, tab=p, n_tok=16, cols=None: L.ldr_read_fwd_any(
        tab, tab, n, p, p, 16, base, null, 0.0, p, n if cols is None else cols, p, n if cols is None else cols, 1.0,
        0.1, p, p, p, null, n_tok, d, 1, null)
    assert rd(0, 64) == -2 and rd(many, 64) == -2 and rd(2, 0) == -2
    assert rd(2, 64, tab=null) == -1 and rd(2, 64, cols=5) == -1
    assert rd(2, 64, base=odd) == -3
    assert rd(70, 100, n_tok=0) == 0 and rd(3, 8200, n_tok=0) == 0 and rd(2, 1, n_tok=0) == 0
    b1 = lambda n, parts=4, wz=p, g=p: L.ldr_read_bwd1_any(
        p, p, n, g, null, p, p, 16, p, p, n, p, n, 1.0, 0.1, p, n, p, 0, wz, 16, p, parts, 100, null, null, 0.0, 16,
        100, 1, null)
    assert b1(many) == -2 and b1(2, parts=0) == -1 and b1(2, wz=4100) == -3 and b1(2, g=odd) == -3
    dv = lambda m, d=100, v=p: L.ldr_dv_assemble_any(p, p, p, m, v, p, null, null, 0.0, 0, p, null, 16, d, 1, null)
    assert dv(many) == -2 and dv(2, d=0) == -2 and dv(2, v=odd) == -3
    assert L.ldr_dv_assemble_any(null, null, null, 2, p, p, null, null, 0.0, 0, p, null, 16, 100, 1, null) == -1
    assert L.ldr_dv_assemble_any(p, p, p, 2, p, p, null, null, 0.0, 3, p, null, 16, 100, 1, null) == -1
    assert L.ldr_read_bwd2_list_any(p, many, 0, p, p, p, 16, 16, 100, 1, null) == -2
    assert L.ldr_read_bwd2_list_any(p, 2, 2, p, p, p, 16, 16, 100, 1, null) == -1
    assert L.ldr_blend_sum_any(p, 0, 0.5, 0, p, 16, 100, 1, null) == -2
    assert L.ldr_blend_sum_any(p, 2, 0.5, 0, odd, 16, 100, 1, null) == -3
    assert L.ldr_blend_sum_any(p, 2, 0.5, 1, p, 0, 100, 1, null) == 0
    assert L.ldr_blend_sum_any(p, 2, 0.5, 5, p, 0, 100, 1, null) == -1
