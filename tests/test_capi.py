"""CPU checks of the C ABI: the library loads, exports every symbol include/*.h
declares, and rejects bad arguments before any launch (no GPU work here)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(kr_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def kq():
    import kriya_q4

    if not os.path.exists(kriya_q4.LIB_PATH):
        kriya_q4.build()
    kriya_q4.lib()
    return kriya_q4


def test_every_declared_symbol_is_exported(kq):
    names = declared_functions()
    assert "kr_q4_linear" in names and "kr_q4_mlp" in names
    missing = [n for n in names if not hasattr(kq.lib(), n)]
    assert not missing, missing


def test_abi_version_and_options(kq):
    L = kq.lib()
    assert L.kr_abi_version() == 1
    assert L.kr_set_option(kq.OPT_GEMV_ROWS_PER_WAVE, 3) == kq.KR_E_INVALID
    assert b"rows per wave" in L.kr_last_error()
    assert L.kr_set_option(999, 1) == kq.KR_E_INVALID
    old = L.kr_get_option(kq.OPT_GEMV_ROWS_PER_WAVE)
    assert L.kr_set_option(kq.OPT_GEMV_ROWS_PER_WAVE, 2) == 0
    assert L.kr_get_option(kq.OPT_GEMV_ROWS_PER_WAVE) == 2
    assert L.kr_set_option(kq.OPT_GEMV_ROWS_PER_WAVE, old) == 0


def _mat(kq, qw=0x10000, sc=0x20000, bi=0x30000, n=8, k=128):
    return kq.kr_q4_matrix(qw, sc, bi, n, k)


def test_linear_argument_checks(kq):
    L = kq.lib()
    x, y = 0x40000, 0x50000
    assert L.kr_q4_linear(None, x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, k=96)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_SHAPE
    assert b"multiple of 64" in L.kr_last_error()
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, k=0)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_SHAPE
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, n=0)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_SHAPE
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, qw=0x10008)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_ALIGN
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, sc=0x20001)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_ALIGN
    assert L.kr_q4_linear(ctypes.byref(_mat(kq, qw=None)), x, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_INVALID
    m = ctypes.byref(_mat(kq))
    assert L.kr_q4_linear(m, x + 8, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_ALIGN
    assert L.kr_q4_linear(m, x, 1, y + 2, kq.DTYPE_F32, 0, None) == kq.KR_E_ALIGN
    assert L.kr_q4_linear(m, x, 1, y, 7, 0, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear(m, x, 1, y, kq.DTYPE_F32, 2, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear(m, None, 1, y, kq.DTYPE_F32, 0, None) == kq.KR_E_INVALID
    # empty batch: nothing to do, nothing launched
    assert L.kr_q4_linear(m, None, 0, None, kq.DTYPE_F32, 0, None) == kq.KR_OK


def test_gate_up_and_mlp_argument_checks(kq):
    L = kq.lib()
    g, u = _mat(kq, n=192, k=128), _mat(kq, n=192, k=128)
    bad_u = _mat(kq, n=128, k=128)
    d = _mat(kq, n=128, k=192)
    x, out = 0x40000, 0x50000
    assert L.kr_q4_gate_up_act(ctypes.byref(g), ctypes.byref(bad_u), x, 1, out, 0, 0, None) == kq.KR_E_SHAPE
    assert L.kr_q4_gate_up_act(ctypes.byref(g), ctypes.byref(u), x, 1, out, 0, 9, None) == kq.KR_E_INVALID
    need = L.kr_q4_mlp_workspace_bytes(4, 128, 192)
    assert need >= 4 * 192 * 2 + 4 * 128 * 4 and need % 256 == 0
    rc = L.kr_q4_mlp(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), x, out, 0, 4, 0, 0x60000, need - 1, None)
    assert rc == kq.KR_E_WORKSPACE
    rc = L.kr_q4_mlp(ctypes.byref(g), ctypes.byref(u), ctypes.byref(bad_u), x, out, 0, 4, 0, 0x60000, need, None)
    assert rc == kq.KR_E_SHAPE
    rc = L.kr_q4_mlp(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), None, out, kq.DTYPE_F32, 4, 0, 0x60000,
                     need, None)
    assert rc == kq.KR_E_INVALID  # an f32 residual needs a separate bf16 input


def test_argmax_workspace_sizes_and_checks(kq):
    """kr_argmax_ws: the workspace holds one (value, index) pair per block of a row; the parts per row
    give every block at least 1024 logits and about 512 blocks in all; short workspaces are refused."""
    L = kq.lib()
    assert L.kr_argmax_workspace_bytes(0, 151936) == 0
    for rows, n, parts in ((1, 151936, 148), (16, 151936, 32), (3, 4097, 4), (1, 100, 1), (600, 151936, 1)):
        need = L.kr_argmax_workspace_bytes(rows, n)
        assert need % 256 == 0 and need >= rows * parts * 8 and need < rows * parts * 8 + 256, (rows, n, need)
    need = L.kr_argmax_workspace_bytes(16, 151936)
    logits, out = 0x40000, 0x50000
    assert L.kr_argmax_ws(logits, 16, 151936, out, 0x60000, need - 1, None) == kq.KR_E_WORKSPACE
    assert L.kr_argmax_ws(logits, 16, 151936, out, None, need, None) == kq.KR_E_WORKSPACE
    assert L.kr_argmax_ws(logits, 16, 151936, out, 0x60004, need, None) == kq.KR_E_ALIGN
    assert L.kr_argmax_ws(None, 16, 151936, out, 0x60000, need, None) == kq.KR_E_INVALID
    assert L.kr_argmax_ws(logits, 16, 0, out, 0x60000, need, None) == kq.KR_E_SHAPE
    assert L.kr_argmax_ws(logits, 0, 151936, out, None, 0, None) == 0


def test_linear_workspace_sizes_and_checks(kq):
    """kr_q4_linear_ws: no workspace at m <= 1; otherwise the ticket words then the split-K partials, growing
    with m (a workspace sized for m serves smaller m); short, missing and misaligned workspaces are refused
    before anything runs."""
    L = kq.lib()
    assert L.kr_q4_linear_workspace_bytes(1, 2048, 11008) == 0
    sizes = [L.kr_q4_linear_workspace_bytes(m, 2048, 11008) for m in (2, 5, 16, 63, 96)]
    assert all(sz % 256 == 0 and sz > 0 for sz in sizes) and sizes == sorted(sizes)
    w = ctypes.byref(_mat(kq, n=2048, k=11008))
    x, y = 0x40000, 0x50000
    need = L.kr_q4_linear_workspace_bytes(16, 2048, 11008)
    assert L.kr_q4_linear_ws(w, x, 16, y, kq.DTYPE_F32, 0, 0x60000, need - 1, None) == kq.KR_E_WORKSPACE
    assert L.kr_q4_linear_ws(w, x, 16, y, kq.DTYPE_F32, 0, None, need, None) == kq.KR_E_WORKSPACE
    assert L.kr_q4_linear_ws(w, x, 16, y, kq.DTYPE_F32, 0, 0x60008, need, None) == kq.KR_E_ALIGN
    assert L.kr_q4_linear_ws(w, x, 16, y, 7, 0, 0x60000, need, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear_ws(w, x, 16, y, kq.DTYPE_F32, 2, 0x60000, need, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear_ws(w, None, 16, y, kq.DTYPE_F32, 0, 0x60000, need, None) == kq.KR_E_INVALID
    assert L.kr_q4_linear_ws(ctypes.byref(_mat(kq, k=96)), x, 16, y, kq.DTYPE_F32, 0, 0x60000, need, None) == \
        kq.KR_E_SHAPE
    assert L.kr_q4_linear_ws(w, x, 0, y, kq.DTYPE_F32, 0, None, 0, None) == kq.KR_OK


def test_format_argument_checks(kq):
    L = kq.lib()
    assert L.kr_q4_from_blocks36(0x1000, 4, 100, 0x2000, 0x3000, 0x4000, None) == kq.KR_E_SHAPE
    assert L.kr_q4_from_blocks36(0x1002, 4, 128, 0x2000, 0x3000, 0x4000, None) == kq.KR_E_ALIGN
    assert L.kr_q4_from_blocks36(None, 4, 128, 0x2000, 0x3000, 0x4000, None) == kq.KR_E_INVALID
    assert L.kr_f16_to_bf16(None, None, 0, None) == kq.KR_OK
    assert L.kr_f16_to_bf16(0x1001, 0x2000, 4, None) == kq.KR_E_ALIGN
    assert L.kr_q4_dequant(ctypes.byref(_mat(kq)), 0x1004, None) == kq.KR_E_ALIGN


def test_moe_argument_checks(kq):
    L = kq.lib()
    p = 0x40000
    # routing: topk in 1..min(E, 16), E <= 256, T * topk <= 16384
    assert L.kr_moe_route(p, 4, 8, 0, 1, p, p, p, p, p, None) == kq.KR_E_INVALID
    assert L.kr_moe_route(p, 4, 8, 9, 1, p, p, p, p, p, None) == kq.KR_E_INVALID
    assert L.kr_moe_route(p, 4, 300, 4, 1, p, p, p, p, p, None) == kq.KR_E_INVALID
    assert L.kr_moe_route(p, 4097, 60, 4, 1, p, p, p, p, p, None) == kq.KR_E_SHAPE
    assert L.kr_moe_route(p + 2, 4, 8, 2, 1, p, p, p, p, p, None) == kq.KR_E_ALIGN
    assert L.kr_moe_scan_scatter(p, 16385, 8, p, p, p, None) == kq.KR_E_SHAPE
    assert L.kr_moe_scan_scatter(p, 4, 0, p, p, p, None) == kq.KR_E_INVALID
    # experts: stacked shapes must agree
    E, H, I = 4, 128, 128
    g, u = _mat(kq, n=E * I, k=H), _mat(kq, n=E * I, k=H)
    d = _mat(kq, n=E * H, k=I)
    need = L.kr_q4_moe_workspace_bytes(2, 2, H, I)
    assert need >= 4 * I * 2 + 4 * H * 4
    args = (p, 2, 2, p, p, p, 0, p, kq.DTYPE_F32, 0, 0x80000, need, None)
    assert L.kr_q4_moe_experts(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), 3, *args) == kq.KR_E_SHAPE
    bad_d = _mat(kq, n=E * H, k=256)
    assert L.kr_q4_moe_experts(ctypes.byref(g), ctypes.byref(u), ctypes.byref(bad_d), E, *args) == kq.KR_E_SHAPE
    short = args[:-2] + (need - 16, None)
    assert L.kr_q4_moe_experts(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), E, *short) == kq.KR_E_WORKSPACE
    wide = _mat(kq, n=E * I, k=8192), _mat(kq, n=E * I, k=8192), _mat(kq, n=E * 8192, k=I)
    assert L.kr_q4_moe_experts(*(ctypes.byref(w) for w in wide), E, *args) == kq.KR_E_UNSUPPORTED
    odd = _mat(kq, n=E * 192, k=H), _mat(kq, n=E * 192, k=H), _mat(kq, n=E * H, k=192)
    assert L.kr_q4_moe_experts(*(ctypes.byref(w) for w in odd), E, *args) == kq.KR_E_UNSUPPORTED


def test_mlp_noalloc_rejects_sizes_beyond_its_scratch(kq):
    """kr_q4_mlp_noalloc checks its need against the library's per-GPU scratch before any HIP call."""
    L = kq.lib()
    assert L.kr_q4_mlp_noalloc_max_bytes() == 4 << 20
    g, u = _mat(kq, n=11008, k=2048), _mat(kq, n=11008, k=2048)
    d = _mat(kq, n=2048, k=11008)
    h = 0x40000
    rc = L.kr_q4_mlp_noalloc(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), None, h, kq.DTYPE_BF16, 64, 0, None)
    assert rc == kq.KR_E_WORKSPACE
    assert b"kr_q4_mlp_noalloc" in L.kr_last_error() and b"kr_q4_mlp with a workspace" in L.kr_last_error()
    assert L.kr_q4_mlp_workspace_bytes(37, 2048, 11008) <= 4 << 20 < L.kr_q4_mlp_workspace_bytes(38, 2048, 11008)


def test_moe_block_argument_checks(kq):
    """kr_q4_moe_block validates all three stages before its first launch (no GPU work here)."""
    L = kq.lib()
    E, H, I = 8, 256, 128
    router = _mat(kq, n=E, k=H)
    g, u = _mat(kq, n=E * I, k=H), _mat(kq, n=E * I, k=H)
    d = _mat(kq, n=E * H, k=I)
    x, y, ws = 0x40000, 0x50000, 0x60000
    big = 1 << 30
    args = lambda r=router, topk=2, act=0, dt=kq.DTYPE_F32: (ctypes.byref(r), ctypes.byref(g), ctypes.byref(u),  # noqa: E731
                                                              ctypes.byref(d), E, x, 4, topk, 1, act, y, dt, 0, ws,
                                                              big, None)
    assert L.kr_q4_moe_block(*args(r=_mat(kq, n=E + 1, k=H))) == kq.KR_E_SHAPE
    assert b"router" in L.kr_last_error()
    assert L.kr_q4_moe_block(*args(topk=0)) == kq.KR_E_INVALID
    assert L.kr_q4_moe_block(*args(topk=17)) == kq.KR_E_INVALID
    assert L.kr_q4_moe_block(*args(act=9)) == kq.KR_E_INVALID
    assert L.kr_q4_moe_block(*args(dt=7)) == kq.KR_E_INVALID
    bad_down = _mat(kq, n=E * H, k=I + 64)
    assert L.kr_q4_moe_block(ctypes.byref(router), ctypes.byref(g), ctypes.byref(u), ctypes.byref(bad_down), E, x, 4,
                             2, 1, 0, y, kq.DTYPE_F32, 0, ws, big, None) == kq.KR_E_SHAPE
    need = L.kr_q4_moe_block_workspace_bytes(4, E, 2, H, I)
    assert need >= L.kr_q4_moe_workspace_bytes(4, 2, H, I)
    assert L.kr_q4_moe_block(ctypes.byref(router), ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), E, x, 4, 2, 1,
                             0, y, kq.DTYPE_F32, 0, ws, need - 1, None) == kq.KR_E_WORKSPACE


def test_every_option_round_trips(kq):
    """Each KR_OPT_* the header declares is known to kr_get_option, and setting its current value back
    succeeds; the few-token and prefill switches reject values outside their ranges."""
    L = kq.lib()
    hdr = open(os.path.join(ROOT, "include", "kriya_q4.h")).read()
    opts = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (KR_OPT_\w+) (\d+)", hdr)}
    assert len(opts) >= 16
    for name, code in opts.items():
        cur = L.kr_get_option(code)
        assert cur >= 0, name
        assert L.kr_set_option(code, cur) == 0, (name, L.kr_last_error())
    for name, bad in (("KR_OPT_SKINNY_GROUPS", 3), ("KR_OPT_SKINNY_DEPTH", 4), ("KR_OPT_SKINNY_DEPTH", 1),
                      ("KR_OPT_PREFILL_OPERANDS", 2), ("KR_OPT_SPLITK_TICKETS", 2)):
        assert L.kr_set_option(opts[name], bad) == kq.KR_E_INVALID, name
    assert L.kr_get_option(opts["KR_OPT_SKINNY_GROUPS"]) == 2
    assert L.kr_get_option(opts["KR_OPT_SKINNY_DEPTH"]) == 0
