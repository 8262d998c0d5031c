"""ctypes wrapper of the CPU oracle (libkr_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.  Only
tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may import
this package; the product library never loads it.

Weights are passed as a ``Q4Planar`` triplet (numpy arrays):
  qw     uint32 [n, k/8]   element 8w+j of a row in bits 4j..4j+3 of word w
  scales uint16 [n, k/64]  bf16 bits
  biases uint16 [n, k/64]  bf16 bits
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkr_oracle.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


def build() -> None:
    """Compile libkr_oracle.so from oracle/kr_oracle.c (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    L.kro_f32_to_bf16.restype = ctypes.c_uint16
    L.kro_f32_to_bf16.argtypes = [ctypes.c_float]
    L.kro_bf16_to_f32.restype = ctypes.c_float
    L.kro_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.kro_f16_to_f32.restype = ctypes.c_float
    L.kro_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.kro_half_to_bf16.restype = ctypes.c_uint16
    L.kro_half_to_bf16.argtypes = [ctypes.c_uint16, ctypes.c_int]
    L.kro_f32_to_bf16_n.argtypes = [_f32p, _u16p, ctypes.c_size_t]
    L.kro_bf16_to_f32_n.argtypes = [_u16p, _f32p, ctypes.c_size_t]
    L.kro_f16_to_f32_n.argtypes = [_u16p, _f32p, ctypes.c_size_t]
    L.kro_quantize_q4_g64.restype = ctypes.c_int
    L.kro_quantize_q4_g64.argtypes = [_f32p, ctypes.c_size_t, _u8p]
    L.kro_dequant_blocks36.argtypes = [_u8p, ctypes.c_size_t, _f32p]
    L.kro_dequant_planar.argtypes = [_u32p, _u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32, _f32p]
    L.kro_blocks36_to_planar.argtypes = [_u8p, ctypes.c_uint32, ctypes.c_uint32, _u32p, _u16p, _u16p]
    L.kro_planar_to_blocks36.argtypes = [_u32p, _u16p, _u16p, ctypes.c_uint32, ctypes.c_uint32, _u8p]
    L.kro_mlx_pack_blocks36.restype = ctypes.c_long
    L.kro_mlx_pack_blocks36.argtypes = [_u8p, ctypes.c_size_t, _u16p, ctypes.c_size_t, ctypes.c_int,
                                        _u16p, ctypes.c_size_t, ctypes.c_int, _u8p]
    L.kro_split_blocks36.argtypes = [_u8p, ctypes.c_size_t, _u8p, _u16p]
    L.kro_join_blocks36.argtypes = [_u8p, _u16p, ctypes.c_size_t, _u8p]
    W = [_u32p, _u16p, _u16p]
    L.kro_q4_matmul.argtypes = W + [ctypes.c_uint32, ctypes.c_uint32, _u16p, ctypes.c_uint32, _f32p, ctypes.c_int]
    L.kro_q4_matmul_f64.argtypes = W + [ctypes.c_uint32, ctypes.c_uint32, _u16p, ctypes.c_uint32, _f64p, ctypes.c_int]
    L.kro_f32_matmul.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _f32p, ctypes.c_uint32, _f32p, ctypes.c_int]
    L.kro_activation.restype = ctypes.c_float
    L.kro_activation.argtypes = [ctypes.c_float, ctypes.c_int]
    L.kro_q4_gate_up_act.argtypes = W + W + [ctypes.c_uint32, ctypes.c_uint32, _u16p, ctypes.c_uint32,
                                             ctypes.c_int, _f32p, ctypes.c_int]
    L.kro_q4_mlp.argtypes = W + W + W + [ctypes.c_uint32, ctypes.c_uint32, _u16p, ctypes.c_uint32,
                                         ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int]
    L.kro_moe_route.restype = ctypes.c_int
    L.kro_moe_route.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                _u32p, _f32p, _u32p, _u32p, _u32p]
    L.kro_moe_scan_scatter.restype = ctypes.c_int
    L.kro_moe_scan_scatter.argtypes = [_u32p, ctypes.c_size_t, ctypes.c_uint32, _u32p, _u32p, _u32p]
    L.kro_moe_experts.argtypes = W + W + W + [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                              _u16p, ctypes.c_uint32, ctypes.c_uint32,
                                              _u32p, _f32p, ctypes.c_int, _f32p, ctypes.c_int]


def _p(arr: np.ndarray, ctype):
    assert arr.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


def default_threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


@dataclass
class Q4Planar:
    """Planar Q4_G64 triplet in host memory."""
    qw: np.ndarray
    scales: np.ndarray
    biases: np.ndarray

    @property
    def n(self) -> int:
        return int(self.qw.shape[0])

    @property
    def k(self) -> int:
        return int(self.qw.shape[1]) * 8

    def ptrs(self):
        return (_p(self.qw, ctypes.c_uint32), _p(self.scales, ctypes.c_uint16), _p(self.biases, ctypes.c_uint16))

    def rows(self, lo: int, hi: int) -> "Q4Planar":
        return Q4Planar(np.ascontiguousarray(self.qw[lo:hi]), np.ascontiguousarray(self.scales[lo:hi]),
                        np.ascontiguousarray(self.biases[lo:hi]))


# ---- scalar / vector conversions ------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().kro_f32_to_bf16_n(_p(x, ctypes.c_float), _p(out, ctypes.c_uint16), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().kro_bf16_to_f32_n(_p(b, ctypes.c_uint16), _p(out, ctypes.c_float), b.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().kro_f16_to_f32_n(_p(h, ctypes.c_uint16), _p(out, ctypes.c_float), h.size)
    return out


def half_to_bf16(raw: int, is_f16: bool) -> int:
    return int(lib().kro_half_to_bf16(raw, int(is_f16)))


# ---- quantize / dequantize / layouts --------------------------------------------

def quantize_q4_g64(w) -> np.ndarray:
    """Returns the 36-byte blocks as uint8 [count/64, 36]; raises on bad length."""
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    out = np.zeros((max(w.size // 64, 1), 36), dtype=np.uint8)
    rc = lib().kro_quantize_q4_g64(_p(w, ctypes.c_float), w.size, _p(out, ctypes.c_uint8))
    if rc != 0:
        raise ValueError(f"ShapeMismatch: {w.size} elements is not a multiple of 64")
    return out[: w.size // 64]


def dequant_blocks36(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 36)
    out = np.empty(blocks.shape[0] * 64, dtype=np.float32)
    lib().kro_dequant_blocks36(_p(blocks, ctypes.c_uint8), blocks.shape[0], _p(out, ctypes.c_float))
    return out


def dequant_planar(w: Q4Planar) -> np.ndarray:
    out = np.empty((w.n, w.k), dtype=np.float32)
    lib().kro_dequant_planar(*w.ptrs(), w.n, w.k, _p(out, ctypes.c_float))
    return out


def blocks36_to_planar(blocks: np.ndarray, n: int, k: int) -> Q4Planar:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 36)
    assert blocks.shape[0] == n * (k // 64)
    w = Q4Planar(np.empty((n, k // 8), np.uint32), np.empty((n, k // 64), np.uint16),
                 np.empty((n, k // 64), np.uint16))
    lib().kro_blocks36_to_planar(_p(blocks, ctypes.c_uint8), n, k, *w.ptrs())
    return w


def planar_to_blocks36(w: Q4Planar) -> np.ndarray:
    out = np.empty((w.n * (w.k // 64), 36), dtype=np.uint8)
    lib().kro_planar_to_blocks36(*w.ptrs(), w.n, w.k, _p(out, ctypes.c_uint8))
    return out


def mlx_pack_blocks36(wbytes: np.ndarray, scales_raw: np.ndarray, s_is_f16: bool,
                      biases_raw: np.ndarray, b_is_f16: bool) -> np.ndarray:
    wbytes = np.ascontiguousarray(wbytes, dtype=np.uint8).ravel()
    s = np.ascontiguousarray(scales_raw, dtype=np.uint16).ravel()
    b = np.ascontiguousarray(biases_raw, dtype=np.uint16).ravel()
    out = np.zeros((max(wbytes.size // 32, 1), 36), dtype=np.uint8)
    rc = lib().kro_mlx_pack_blocks36(_p(wbytes, ctypes.c_uint8), wbytes.size, _p(s, ctypes.c_uint16), s.size,
                                     int(s_is_f16), _p(b, ctypes.c_uint16), b.size, int(b_is_f16),
                                     _p(out, ctypes.c_uint8))
    if rc == -1:
        raise ValueError("InvalidMetadata: weight byte length is not a multiple of 32")
    if rc == -2:
        raise ValueError("ShapeMismatch: scale/bias count does not match block count")
    return out[:rc]


def split_blocks36(blocks: np.ndarray):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 36)
    nb = blocks.shape[0]
    qs = np.empty((nb, 32), np.uint8)
    sb = np.empty((nb, 2), np.uint16)
    lib().kro_split_blocks36(_p(blocks, ctypes.c_uint8), nb, _p(qs, ctypes.c_uint8), _p(sb, ctypes.c_uint16))
    return qs, sb


def join_blocks36(qs: np.ndarray, sb: np.ndarray) -> np.ndarray:
    qs = np.ascontiguousarray(qs, dtype=np.uint8).reshape(-1, 32)
    sb = np.ascontiguousarray(sb, dtype=np.uint16).reshape(-1, 2)
    out = np.empty((qs.shape[0], 36), np.uint8)
    lib().kro_join_blocks36(_p(qs, ctypes.c_uint8), _p(sb, ctypes.c_uint16), qs.shape[0], _p(out, ctypes.c_uint8))
    return out


# ---- matmul family -----------------------------------------------------------

def _x(x_bf16: np.ndarray, k: int):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    assert x.size % k == 0
    return x, x.size // k


def q4_matmul(w: Q4Planar, x_bf16: np.ndarray, threads: int | None = None) -> np.ndarray:
    """Y[m, n] = sequential f32 dot of dequantized W rows with bf16 X rows."""
    x, m = _x(x_bf16, w.k)
    y = np.empty((m, w.n), np.float32)
    lib().kro_q4_matmul(*w.ptrs(), w.n, w.k, _p(x, ctypes.c_uint16), m, _p(y, ctypes.c_float),
                        threads or default_threads())
    return y


def q4_matmul_f64(w: Q4Planar, x_bf16: np.ndarray, threads: int | None = None) -> np.ndarray:
    x, m = _x(x_bf16, w.k)
    y = np.empty((m, w.n), np.float64)
    lib().kro_q4_matmul_f64(*w.ptrs(), w.n, w.k, _p(x, ctypes.c_uint16), m, _p(y, ctypes.c_double),
                            threads or default_threads())
    return y


def f32_matmul(w_f32: np.ndarray, x_f32: np.ndarray, threads: int | None = None) -> np.ndarray:
    """Y[m, n] = sequential f32 dot of pre-dequantised rows w [n, k] with x [m, k] (f32)."""
    w = np.ascontiguousarray(w_f32, dtype=np.float32)
    n, k = w.shape
    x = np.ascontiguousarray(x_f32, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), np.float32)
    lib().kro_f32_matmul(_p(w, ctypes.c_float), n, k, _p(x, ctypes.c_float), x.shape[0], _p(y, ctypes.c_float),
                         threads or default_threads())
    return y


def activation(g: float, variant: int) -> float:
    return float(lib().kro_activation(g, variant))


def q4_gate_up_act(gate: Q4Planar, up: Q4Planar, x_bf16: np.ndarray, variant: int = 0,
                   threads: int | None = None) -> np.ndarray:
    x, m = _x(x_bf16, gate.k)
    a = np.empty((m, gate.n), np.float32)
    lib().kro_q4_gate_up_act(*gate.ptrs(), *up.ptrs(), gate.n, gate.k, _p(x, ctypes.c_uint16), m, variant,
                             _p(a, ctypes.c_float), threads or default_threads())
    return a


def q4_mlp(gate: Q4Planar, up: Q4Planar, down: Q4Planar, x_bf16: np.ndarray, variant: int = 0,
           bf16_intermediate: bool = True, threads: int | None = None) -> np.ndarray:
    """down . act(gate x) * (up x), without the residual add; f32 [m, hidden]."""
    x, m = _x(x_bf16, gate.k)
    y = np.empty((m, down.n), np.float32)
    lib().kro_q4_mlp(*gate.ptrs(), *up.ptrs(), *down.ptrs(), down.n, gate.n, _p(x, ctypes.c_uint16), m,
                     variant, int(bf16_intermediate), _p(y, ctypes.c_float), threads or default_threads())
    return y


def moe_route(logits: np.ndarray, topk: int, normalize: bool = True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    experts = np.empty((T, topk), np.uint32)
    weights = np.empty((T, topk), np.float32)
    counts = np.empty(E, np.uint32)
    offsets = np.empty(E + 1, np.uint32)
    sorted_assign = np.empty(max(T * topk, 1), np.uint32)
    rc = lib().kro_moe_route(_p(logits, ctypes.c_float), T, E, topk, int(normalize),
                             _p(experts, ctypes.c_uint32), _p(weights, ctypes.c_float),
                             _p(counts, ctypes.c_uint32), _p(offsets, ctypes.c_uint32),
                             _p(sorted_assign, ctypes.c_uint32))
    if rc != 0:
        raise ValueError("invalid top-k")
    return experts, weights, counts, offsets, sorted_assign[: T * topk]


def moe_scan_scatter(experts: np.ndarray, num_experts: int):
    experts = np.ascontiguousarray(experts, dtype=np.uint32).ravel()
    counts = np.empty(num_experts, np.uint32)
    offsets = np.empty(num_experts + 1, np.uint32)
    sorted_assign = np.empty(max(experts.size, 1), np.uint32)
    rc = lib().kro_moe_scan_scatter(_p(experts, ctypes.c_uint32), experts.size, num_experts,
                                    _p(counts, ctypes.c_uint32), _p(offsets, ctypes.c_uint32),
                                    _p(sorted_assign, ctypes.c_uint32))
    if rc != 0:
        raise ValueError("expert id out of range")
    return counts, offsets, sorted_assign[: experts.size]


def moe_experts(gate: Q4Planar, up: Q4Planar, down: Q4Planar, num_experts: int, x_bf16: np.ndarray,
                experts: np.ndarray, weights: np.ndarray, variant: int = 0,
                threads: int | None = None) -> np.ndarray:
    hidden = gate.k
    inter = gate.n // num_experts
    x, T = _x(x_bf16, hidden)
    experts = np.ascontiguousarray(experts, dtype=np.uint32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    K = experts.size // max(T, 1) if T else 0
    y = np.empty((T, hidden), np.float32)
    lib().kro_moe_experts(*gate.ptrs(), *up.ptrs(), *down.ptrs(), num_experts, hidden, inter,
                          _p(x, ctypes.c_uint16), T, K, _p(experts, ctypes.c_uint32),
                          _p(weights, ctypes.c_float), variant, _p(y, ctypes.c_float),
                          threads or default_threads())
    return y
