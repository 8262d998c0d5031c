"""Python binding of libkriya_q4.so (the C ABI in include/kriya_q4.h).

Device memory and streams come from PyTorch (plumbing only): every call passes
raw device pointers and the current HIP stream to the C ABI, which launches
the gfx950 kernels.  There is no fallback: if the library is missing or no GPU
is present, calls raise.

Names mirror kriya-rt's operator surface (crates/kriya-backend-metal/src/
encoder.rs): ``encode_q4_linear`` (:2361), ``encode_q4_linear_accumulate``
(:2497), ``encode_fused_gate_up`` (:2703), ``encode_dense_mlp`` (:2851).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np
import torch  # must be imported before the library: it loads the HIP runtime both share

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("KRIYA_Q4_LIB") or os.path.join(_PKG_DIR, "libkriya_q4.so")

# C ABI constants (include/kriya_q4.h)
KR_OK = 0
KR_E_INVALID, KR_E_SHAPE, KR_E_ALIGN, KR_E_HIP, KR_E_WORKSPACE, KR_E_UNSUPPORTED = -1, -2, -3, -4, -5, -6
DTYPE_BF16, DTYPE_F32 = 0, 1
ACT_SWIGLU, ACT_GEGLU, ACT_RELU = 0, 1, 2
OPT_GEMV_ROWS_PER_WAVE, OPT_GEMV_MAX_BLOCKS, OPT_GEMV_SPLIT_K_CHUNKS = 1, 2, 3
OPT_GEMV_BLOCK_ROWS, OPT_GEMV_PERSISTENT_BLOCKS, OPT_SKINNY_MAX_BLOCKS, OPT_PREFILL_KERNEL = 4, 5, 6, 7
OPT_GEMV_LONG_ROWS = 8
OPT_GEMV_TOKENS = 9
OPT_MOE_GEMV = 10
OPT_GEMV_LONG_GROUPS = 11
OPT_SPLITK_TICKETS = 12
OPT_ATTN_MERGE_WAVE = 13
OPT_PREFILL_OPERANDS = 14
OPT_SKINNY_GROUPS = 15
OPT_SKINNY_DEPTH = 16
OPT_MOE_COMBINE = 17
OPT_MOE_ROUTE_FUSED = 18
OPT_PREFILL_XCD_SPLIT = 19
OPT_ATTN_SLICE64 = 20
OPT_ATTN_MERGE_OPROJ = 21

_lib = None


class KrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"kriya_q4 error {code}: {msg}")
        self.code = code


class kr_q4_matrix(ctypes.Structure):
    _fields_ = [("qw", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("n", ctypes.c_uint32), ("k", ctypes.c_uint32)]


def build() -> None:
    """Compile libkriya_q4.so with hipcc for gfx950 (in-tree)."""
    subprocess.run(["make", "-s", "-C", _PKG_DIR, f"-j{min(os.cpu_count() or 1, 16)}"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        M = ctypes.POINTER(kr_q4_matrix)
        vp, u32, i32, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t
        sig = {
            "kr_abi_version": (i32, []),
            "kr_last_error": (ctypes.c_char_p, []),
            "kr_set_option": (i32, [i32, i32]),
            "kr_get_option": (i32, [i32]),
            "kr_q4_dequant": (i32, [M, vp, vp]),
            "kr_stream_read_pieces": (sz, [sz]),
            "kr_stream_read": (i32, [vp, sz, u32, vp, vp]),
            "kr_q4_from_blocks36": (i32, [vp, u32, u32, vp, vp, vp, vp]),
            "kr_q4_to_blocks36": (i32, [M, vp, vp]),
            "kr_q4_from_split": (i32, [vp, vp, u32, u32, vp, vp, vp, vp]),
            "kr_q4_to_split": (i32, [M, vp, vp, vp]),
            "kr_f16_to_bf16": (i32, [vp, vp, sz, vp]),
            "kr_q4_linear": (i32, [M, vp, u32, vp, i32, i32, vp]),
            "kr_q4_linear_workspace_bytes": (sz, [u32, u32, u32]),
            "kr_q4_linear_ws": (i32, [M, vp, u32, vp, i32, i32, vp, sz, vp]),
            "kr_q4_gate_up_act": (i32, [M, M, vp, u32, vp, i32, i32, vp]),
            "kr_q4_mlp_workspace_bytes": (sz, [u32, u32, u32]),
            "kr_q4_qkv": (i32, [M, M, M, vp, vp, vp, vp, u32, vp, vp, vp, i32, vp]),
            "kr_q4_mlp": (i32, [M, M, M, vp, vp, i32, u32, i32, vp, sz, vp]),
            "kr_q4_mlp_noalloc_max_bytes": (sz, []),
            "kr_q4_mlp_noalloc": (i32, [M, M, M, vp, vp, i32, u32, i32, vp]),
            "kr_moe_route": (i32, [vp, u32, u32, u32, i32, vp, vp, vp, vp, vp, vp]),
            "kr_moe_scan_scatter": (i32, [vp, u32, u32, vp, vp, vp, vp]),
            "kr_q4_moe_workspace_bytes": (sz, [u32, u32, u32, u32]),
            "kr_q4_moe_experts": (i32, [M, M, M, u32, vp, u32, u32, vp, vp, vp, i32, vp, i32, i32, vp, sz, vp]),
            "kr_q4_moe_route_experts": (i32, [M, M, M, u32, vp, u32, u32, vp, i32, vp, vp, vp, vp, vp, i32, vp, i32,
                                              i32, vp, sz, vp]),
            "kr_q4_moe_block_workspace_bytes": (sz, [u32, u32, u32, u32, u32]),
            "kr_q4_moe_block": (i32, [M, M, M, M, u32, vp, u32, u32, i32, i32, vp, i32, i32, vp, sz, vp]),
            "kr_q4_embedding": (i32, [M, vp, u32, vp, vp]),
            "kr_rmsnorm": (i32, [vp, vp, u32, u32, ctypes.c_float, vp, vp]),
            "kr_rope_kv_append": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp, u32, vp]),
            "kr_attention_decode": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp, vp]),
            "kr_argmax": (i32, [vp, u32, u32, vp, vp]),
            "kr_argmax_workspace_bytes": (sz, [u32, u32]),
            "kr_argmax_ws": (i32, [vp, u32, u32, vp, vp, sz, vp]),
            "kr_attention_workspace_bytes": (sz, [u32, u32, u32, u32]),
            "kr_rmsnorm_q4_qkv": (i32, [vp, vp, ctypes.c_float, M, M, M, vp, vp, vp, u32, vp, vp, vp, i32, vp, vp]),
            "kr_rmsnorm_q4_mlp_workspace_bytes": (sz, [u32, u32, u32]),
            "kr_rmsnorm_q4_mlp": (i32, [M, M, M, vp, vp, ctypes.c_float, u32, i32, vp, sz, vp]),
            "kr_rope_attention_decode": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp, u32, vp, vp, sz, vp]),
            "kr_attention_q4_out_workspace_bytes": (sz, [u32, u32, u32, u32]),
            "kr_rope_attention_q4_out": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp, u32, M, vp, i32, vp, sz,
                                               vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != KR_OK:
        raise KrError(rc, lib().kr_last_error().decode())


def _stream(stream) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    return t.data_ptr()


def set_option(option: int, value: int) -> None:
    _check(lib().kr_set_option(option, value))


def get_option(option: int) -> int:
    return int(lib().kr_get_option(option))


class Q4Matrix:
    """Planar Q4_G64 weights resident on the GPU.

    qw int32 [n, k/8] (u32 bits), scales/biases int16 [n, k/64] (bf16 bits).
    """

    def __init__(self, qw: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor):
        self.qw, self.scales, self.biases = qw, scales, biases
        self.n = int(qw.shape[0])
        self.k = int(qw.shape[1]) * 8
        self._desc = kr_q4_matrix(qw.data_ptr(), scales.data_ptr(), biases.data_ptr(), self.n, self.k)

    @classmethod
    def from_numpy(cls, qw: np.ndarray, scales: np.ndarray, biases: np.ndarray, device="cuda") -> "Q4Matrix":
        def up(a, dt):
            return torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(device)
        return cls(up(qw, np.int32), up(scales, np.int16), up(biases, np.int16))

    @classmethod
    def empty(cls, n: int, k: int, device="cuda") -> "Q4Matrix":
        return cls(torch.empty((n, k // 8), dtype=torch.int32, device=device),
                   torch.empty((n, k // 64), dtype=torch.int16, device=device),
                   torch.empty((n, k // 64), dtype=torch.int16, device=device))

    @classmethod
    def from_blocks36(cls, blocks: torch.Tensor, n: int, k: int, stream=None) -> "Q4Matrix":
        """36-byte BlockQ4Group64 blocks (uint8 device tensor) -> planar, on the GPU."""
        w = cls.empty(n, k, device=blocks.device)
        _check(lib().kr_q4_from_blocks36(_ptr(blocks), n, k, _ptr(w.qw), _ptr(w.scales), _ptr(w.biases),
                                         _stream(stream)))
        return w

    def to_blocks36(self, stream=None) -> torch.Tensor:
        out = torch.empty(self.n * (self.k // 64) * 36, dtype=torch.uint8, device=self.qw.device)
        _check(lib().kr_q4_to_blocks36(ctypes.byref(self._desc), _ptr(out), _stream(stream)))
        return out

    @classmethod
    def from_split(cls, qs: torch.Tensor, sb: torch.Tensor, n: int, k: int, in_place: bool = False,
                   stream=None) -> "Q4Matrix":
        """Split planes (32-byte nibble blocks, {scale, bias} bf16 pairs; uint8 device tensors) -> planar.
        in_place: the nibble plane becomes qw itself (no copy)."""
        w = cls.empty(n, k, device=qs.device)
        if in_place:
            w = cls(qs.view(torch.int32).view(n, k // 8), w.scales, w.biases)
        _check(lib().kr_q4_from_split(_ptr(qs), _ptr(sb), n, k, _ptr(w.qw), _ptr(w.scales), _ptr(w.biases),
                                      _stream(stream)))
        return w

    def to_split(self, stream=None):
        """Planar -> (nibble plane, {scale, bias} plane) as uint8 device tensors."""
        nb = self.n * (self.k // 64)
        qs = torch.empty(nb * 32, dtype=torch.uint8, device=self.qw.device)
        sb = torch.empty(nb * 4, dtype=torch.uint8, device=self.qw.device)
        _check(lib().kr_q4_to_split(ctypes.byref(self._desc), _ptr(qs), _ptr(sb), _stream(stream)))
        return qs, sb

    def rows(self, lo: int, hi: int) -> "Q4Matrix":
        return Q4Matrix(self.qw[lo:hi], self.scales[lo:hi], self.biases[lo:hi])

    @property
    def desc(self):
        return ctypes.byref(self._desc)

    def nbytes(self) -> int:
        return self.qw.numel() * 4 + self.scales.numel() * 2 + self.biases.numel() * 2


def _out_dtype(dt: int):
    return torch.float32 if dt == DTYPE_F32 else torch.bfloat16


def _dt_of(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype in (torch.bfloat16, torch.int16):
        return DTYPE_BF16
    raise ValueError(f"unsupported dtype {t.dtype}")


def dequant(w: Q4Matrix, stream=None) -> torch.Tensor:
    out = torch.empty((w.n, w.k), dtype=torch.float32, device=w.qw.device)
    _check(lib().kr_q4_dequant(w.desc, _ptr(out), _stream(stream)))
    return out


def f16_to_bf16(t: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    out = torch.empty_like(t) if out is None else out
    _check(lib().kr_f16_to_bf16(_ptr(t), _ptr(out), t.numel(), _stream(stream)))
    return out


def q4_linear(w: Q4Matrix, x: torch.Tensor, y: Optional[torch.Tensor] = None, out_dtype: int = DTYPE_F32,
              accumulate: bool = False, workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """y[m, n] (=|+=) x[m, k] @ W^T.  x is bf16 [m, k] (or [k]).  With a workspace (linear_workspace),
    kr_q4_linear_ws: a few tokens over a long K split K over blocks."""
    m = x.numel() // w.k
    if y is None:
        y = torch.zeros((m, w.n), dtype=_out_dtype(out_dtype), device=x.device)
    if workspace is None:
        _check(lib().kr_q4_linear(w.desc, _ptr(x), m, _ptr(y), _dt_of(y), int(accumulate), _stream(stream)))
    else:
        _check(lib().kr_q4_linear_ws(w.desc, _ptr(x), m, _ptr(y), _dt_of(y), int(accumulate), _ptr(workspace),
                                     workspace.numel(), _stream(stream)))
    return y


def linear_workspace_bytes(m: int, n: int, k: int) -> int:
    return int(lib().kr_q4_linear_workspace_bytes(m, n, k))


def linear_workspace(m: int, n: int, k: int, device="cuda") -> torch.Tensor:
    """Device workspace of kr_q4_linear_ws (split-K partials and the counters, which must start at zero: the
    call leaves them zero)."""
    return torch.zeros(max(linear_workspace_bytes(m, n, k), 16), dtype=torch.uint8, device=device)


def gate_up_act(gate: Q4Matrix, up: Q4Matrix, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                out_dtype: int = DTYPE_F32, activation: int = ACT_SWIGLU, stream=None) -> torch.Tensor:
    m = x.numel() // gate.k
    if out is None:
        out = torch.empty((m, gate.n), dtype=_out_dtype(out_dtype), device=x.device)
    _check(lib().kr_q4_gate_up_act(gate.desc, up.desc, _ptr(x), m, _ptr(out), _dt_of(out), activation,
                                   _stream(stream)))
    return out


def mlp_workspace_bytes(m: int, hidden: int, intermediate: int) -> int:
    return int(lib().kr_q4_mlp_workspace_bytes(m, hidden, intermediate))


def mlp_workspace(m: int, hidden: int, intermediate: int, device="cuda") -> torch.Tensor:
    """Device workspace of an MLP call (bf16 intermediate, split-K partials and their counters, which
    must start at zero: the call leaves them zero)."""
    return torch.zeros(mlp_workspace_bytes(m, hidden, intermediate), dtype=torch.uint8, device=device)


def qkv(q: Q4Matrix, k: Q4Matrix, v: Q4Matrix, x: torch.Tensor, q_bias=None, k_bias=None, v_bias=None,
        out_dtype: int = DTYPE_F32, outs=None, stream=None):
    """(x q^T + q_bias, x k^T + k_bias, x v^T + v_bias) for x bf16 [m, hidden]."""
    m = x.numel() // q.k
    if outs is None:
        outs = tuple(torch.empty((m, w.n), dtype=_out_dtype(out_dtype), device=x.device) for w in (q, k, v))
    _check(lib().kr_q4_qkv(q.desc, k.desc, v.desc, _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(x), m,
                           _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]), _dt_of(outs[0]), _stream(stream)))
    return outs


def mlp(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, h: torch.Tensor, x: Optional[torch.Tensor] = None,
        activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """h += down(act(gate x) * (up x)) in place; x defaults to h (bf16 h)."""
    m = h.numel() // down.n
    if workspace is None:
        workspace = mlp_workspace(m, gate.k, gate.n, device=h.device)
    _check(lib().kr_q4_mlp(gate.desc, up.desc, down.desc, _ptr(x), _ptr(h), _dt_of(h), m, activation,
                           _ptr(workspace), workspace.numel(), _stream(stream)))
    return h


def mlp_noalloc(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, h: torch.Tensor, x: Optional[torch.Tensor] = None,
                activation: int = ACT_SWIGLU, stream=None) -> torch.Tensor:
    """mlp() with the library's own per-GPU scratch as the workspace (kr_q4_mlp_noalloc): nothing is
    allocated; calls that overlap on one GPU race."""
    m = h.numel() // down.n
    _check(lib().kr_q4_mlp_noalloc(gate.desc, up.desc, down.desc, _ptr(x), _ptr(h), _dt_of(h), m, activation,
                                   _stream(stream)))
    return h


def rmsnorm_qkv(h: torch.Tensor, ln_weight: torch.Tensor, eps: float, q: Q4Matrix, k: Q4Matrix, v: Q4Matrix,
                q_bias=None, k_bias=None, v_bias=None, out_dtype: int = DTYPE_F32, outs=None,
                xnorm: Optional[torch.Tensor] = None, stream=None):
    """qkv(rmsnorm(h)): the norm fused into the QKV GEMV at m == 1 (xnorm, bf16 [m, k], is needed for m > 1)."""
    m = h.numel() // q.k
    if outs is None:
        outs = tuple(torch.empty((m, w.n), dtype=_out_dtype(out_dtype), device=h.device) for w in (q, k, v))
    if xnorm is None and m > 1:
        xnorm = torch.empty((m, q.k), dtype=torch.bfloat16, device=h.device)
    _check(lib().kr_rmsnorm_q4_qkv(_ptr(h), _ptr(ln_weight), eps, q.desc, k.desc, v.desc, _ptr(q_bias), _ptr(k_bias),
                                   _ptr(v_bias), m, _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]), _dt_of(outs[0]),
                                   _ptr(xnorm), _stream(stream)))
    return outs


def rmsnorm_mlp_workspace(m: int, hidden: int, intermediate: int, device="cuda") -> torch.Tensor:
    nbytes = int(lib().kr_rmsnorm_q4_mlp_workspace_bytes(m, hidden, intermediate))
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)  # zero counters, as mlp_workspace


def rmsnorm_mlp(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, h: torch.Tensor, ln_weight: torch.Tensor, eps: float,
                activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """h += mlp(rmsnorm(h)) in place for bf16 h."""
    m = h.numel() // down.n
    if workspace is None:
        workspace = rmsnorm_mlp_workspace(m, gate.k, gate.n, device=h.device)
    _check(lib().kr_rmsnorm_q4_mlp(gate.desc, up.desc, down.desc, _ptr(h), _ptr(ln_weight), eps, m, activation,
                                   _ptr(workspace), workspace.numel(), _stream(stream)))
    return h


class MoeRoute:
    """Device routing of one MoE step (kr_moe_route outputs)."""

    def __init__(self, tokens: int, experts: int, topk: int, device="cuda"):
        self.tokens, self.experts, self.topk = tokens, experts, topk
        self.selected = torch.empty((tokens, topk), dtype=torch.int32, device=device)
        self.weights = torch.empty((tokens, topk), dtype=torch.float32, device=device)
        self.counts = torch.empty(experts, dtype=torch.int32, device=device)
        self.offsets = torch.empty(experts + 1, dtype=torch.int32, device=device)
        self.sorted_assign = torch.empty(max(tokens * topk, 1), dtype=torch.int32, device=device)


def moe_route(logits: torch.Tensor, topk: int, normalize: bool = True, out: Optional[MoeRoute] = None,
              stream=None) -> MoeRoute:
    """Softmax + top-k + deterministic scan/scatter of f32 logits [tokens, experts]."""
    tokens, experts = logits.shape
    if out is None:
        out = MoeRoute(tokens, experts, topk, device=logits.device)
    _check(lib().kr_moe_route(_ptr(logits), tokens, experts, topk, int(normalize), _ptr(out.selected),
                              _ptr(out.weights), _ptr(out.counts), _ptr(out.offsets), _ptr(out.sorted_assign),
                              _stream(stream)))
    return out


def moe_scan_scatter(selected: torch.Tensor, experts: int, stream=None):
    """(counts, offsets, sorted_assign) of given int32 expert ids."""
    n = selected.numel()
    counts = torch.empty(experts, dtype=torch.int32, device=selected.device)
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=selected.device)
    sorted_assign = torch.empty(max(n, 1), dtype=torch.int32, device=selected.device)
    _check(lib().kr_moe_scan_scatter(_ptr(selected), n, experts, _ptr(counts), _ptr(offsets), _ptr(sorted_assign),
                                     _stream(stream)))
    return counts, offsets, sorted_assign[:n]


def moe_workspace_bytes(tokens: int, topk: int, hidden: int, inter: int) -> int:
    return int(lib().kr_q4_moe_workspace_bytes(tokens, topk, hidden, inter))


def moe_workspace(tokens: int, topk: int, hidden: int, inter: int, device="cuda") -> torch.Tensor:
    return torch.empty(max(moe_workspace_bytes(tokens, topk, hidden, inter), 16), dtype=torch.uint8, device=device)


def moe_experts(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, experts: int, x: torch.Tensor, route: MoeRoute,
                y: Optional[torch.Tensor] = None, out_dtype: int = DTYPE_F32, accumulate: bool = False,
                activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """y[t] (+)= sum_k w[t,k] * down_e(act(gate_e x_t) * up_e x_t) over the routed experts."""
    tokens = route.tokens
    if y is None:
        y = torch.zeros((tokens, gate.k), dtype=_out_dtype(out_dtype), device=x.device)
    if workspace is None:
        workspace = moe_workspace(tokens, route.topk, gate.k, gate.n // experts, device=x.device)
    _check(lib().kr_q4_moe_experts(gate.desc, up.desc, down.desc, experts, _ptr(x), tokens, route.topk,
                                   _ptr(route.weights), _ptr(route.offsets), _ptr(route.sorted_assign), activation,
                                   _ptr(y), _dt_of(y), int(accumulate), _ptr(workspace), workspace.numel(),
                                   _stream(stream)))
    return y


def moe_route_experts(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, experts: int, x: torch.Tensor,
                      logits: torch.Tensor, topk: int, normalize: bool = True, out: Optional[MoeRoute] = None,
                      y: Optional[torch.Tensor] = None, out_dtype: int = DTYPE_F32, accumulate: bool = False,
                      activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None, stream=None):
    """moe_route(logits) then moe_experts in one call (kr_q4_moe_route_experts); returns (y, route)."""
    tokens = int(logits.shape[0])
    if out is None:
        out = MoeRoute(tokens, experts, topk, device=logits.device)
    if y is None:
        y = torch.zeros((tokens, gate.k), dtype=_out_dtype(out_dtype), device=x.device)
    if workspace is None:
        workspace = moe_workspace(tokens, topk, gate.k, gate.n // experts, device=x.device)
    _check(lib().kr_q4_moe_route_experts(gate.desc, up.desc, down.desc, experts, _ptr(x), tokens, topk, _ptr(logits),
                                         int(normalize), _ptr(out.selected), _ptr(out.weights), _ptr(out.counts),
                                         _ptr(out.offsets), _ptr(out.sorted_assign), activation, _ptr(y), _dt_of(y),
                                         int(accumulate), _ptr(workspace), workspace.numel(), _stream(stream)))
    return y, out


def moe_block_workspace(tokens: int, experts: int, topk: int, hidden: int, inter: int, device="cuda") -> torch.Tensor:
    nbytes = int(lib().kr_q4_moe_block_workspace_bytes(tokens, experts, topk, hidden, inter))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def moe_block(router: Q4Matrix, gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, experts: int, x: torch.Tensor,
              topk: int, normalize: bool = True, y: Optional[torch.Tensor] = None, out_dtype: int = DTYPE_F32,
              accumulate: bool = False, activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None,
              stream=None) -> torch.Tensor:
    """The routed MoE stage on the device: f32 router logits (Q4 GEMV) -> routing -> experts -> combine."""
    tokens = x.numel() // gate.k
    if y is None:
        y = torch.zeros((tokens, gate.k), dtype=_out_dtype(out_dtype), device=x.device)
    if workspace is None:
        workspace = moe_block_workspace(tokens, experts, topk, gate.k, gate.n // experts, device=x.device)
    _check(lib().kr_q4_moe_block(router.desc, gate.desc, up.desc, down.desc, experts, _ptr(x), tokens, topk,
                                 int(normalize), activation, _ptr(y), _dt_of(y), int(accumulate), _ptr(workspace),
                                 workspace.numel(), _stream(stream)))
    return y


def embedding(w: Q4Matrix, tokens: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """bf16 rows of the Q4 table for int32 token ids (transformer_glue.metal:122-152)."""
    count = tokens.numel()
    if out is None:
        out = torch.empty((count, w.k), dtype=torch.bfloat16, device=tokens.device)
    _check(lib().kr_q4_embedding(w.desc, _ptr(tokens), count, _ptr(out), _stream(stream)))
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: Optional[torch.Tensor] = None,
            stream=None) -> torch.Tensor:
    dim = weight.numel()
    rows = x.numel() // dim
    if out is None:
        out = torch.empty_like(x)
    _check(lib().kr_rmsnorm(_ptr(x), _ptr(weight), rows, dim, eps, _ptr(out), _stream(stream)))
    return out


def rope_kv_append(q, k, v, cos_sin, positions, q_heads, kv_heads, head_dim, k_cache, v_cache, stream=None):
    batch = positions.numel()
    max_ctx = k_cache.shape[1]
    _check(lib().kr_rope_kv_append(_ptr(q), _ptr(k), _ptr(v), _ptr(cos_sin), _ptr(positions), batch, q_heads,
                                   kv_heads, head_dim, _ptr(k_cache), _ptr(v_cache), max_ctx, _stream(stream)))


def attention_decode(q, k_cache, v_cache, positions, q_heads, kv_heads, head_dim, out=None, stream=None):
    batch = positions.numel()
    max_ctx = k_cache.shape[1]
    if out is None:
        out = torch.empty((batch, q_heads * head_dim), dtype=torch.bfloat16, device=q.device)
    _check(lib().kr_attention_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(positions), batch, q_heads,
                                     kv_heads, head_dim, max_ctx, _ptr(out), _stream(stream)))
    return out


def attention_workspace(batch, q_heads, head_dim, max_ctx, device="cuda") -> torch.Tensor:
    """Device workspace of rope_attention_decode (per-slice partial sums)."""
    nbytes = int(lib().kr_attention_workspace_bytes(batch, q_heads, head_dim, max_ctx))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def rope_attention_decode(q, k, v, cos_sin, positions, q_heads, kv_heads, head_dim, k_cache, v_cache, out=None,
                          workspace=None, stream=None):
    """RoPE + KV append + decode attention (q is read, not rotated in place)."""
    batch = positions.numel()
    max_ctx = k_cache.shape[1]
    if out is None:
        out = torch.empty((batch, q_heads * head_dim), dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = attention_workspace(batch, q_heads, head_dim, max_ctx, device=q.device)
    _check(lib().kr_rope_attention_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(cos_sin), _ptr(positions), batch, q_heads,
                                          kv_heads, head_dim, _ptr(k_cache), _ptr(v_cache), max_ctx, _ptr(out),
                                          _ptr(workspace), workspace.numel() * workspace.element_size(),
                                          _stream(stream)))
    return out


def attention_q4_out_workspace(batch, q_heads, head_dim, max_ctx, device="cuda") -> torch.Tensor:
    n = int(lib().kr_attention_q4_out_workspace_bytes(batch, q_heads, head_dim, max_ctx))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def rope_attention_q4_out(q, k, v, cos_sin, positions, q_heads, kv_heads, head_dim, k_cache, v_cache,
                          o_proj: "Q4Matrix", h: torch.Tensor, workspace=None, stream=None) -> torch.Tensor:
    """h += rope_attention_decode(...) . o_proj^T (kr_rope_attention_q4_out); h bf16 or f32 [batch, n]."""
    batch = int(positions.numel())
    max_ctx = int(k_cache.shape[1])
    if workspace is None:
        workspace = attention_q4_out_workspace(batch, q_heads, head_dim, max_ctx, device=q.device)
    _check(lib().kr_rope_attention_q4_out(_ptr(q), _ptr(k), _ptr(v), _ptr(cos_sin), _ptr(positions), batch, q_heads,
                                          kv_heads, head_dim, _ptr(k_cache), _ptr(v_cache), max_ctx, o_proj.desc,
                                          _ptr(h), _dt_of(h), _ptr(workspace), workspace.numel(), _stream(stream)))
    return h


def argmax_workspace(rows: int, n: int, device="cuda") -> torch.Tensor:
    """Device workspace of argmax(..., workspace=) (per-block partial results)."""
    nbytes = int(lib().kr_argmax_workspace_bytes(rows, n))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def argmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
           stream=None) -> torch.Tensor:
    """Greedy argmax per row (ties to the lowest index, NaN never taken): kr_argmax, or with a workspace
    (argmax_workspace) kr_argmax_ws, which spreads each row over several blocks (same result)."""
    rows, n = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    if workspace is None:
        _check(lib().kr_argmax(_ptr(logits), rows, n, _ptr(out), _stream(stream)))
    else:
        _check(lib().kr_argmax_ws(_ptr(logits), rows, n, _ptr(out), _ptr(workspace), workspace.numel(),
                                  _stream(stream)))
    return out


def stream_read(buf: torch.Tensor, match: int = 0x9E3779B9, hits: Optional[torch.Tensor] = None,
                stream=None) -> torch.Tensor:
    """Measurement helper (no reference counterpart): a plain read of buf's bytes.  hits[i] (int32) is set
    to 1 where some 16-byte unit of the i-th 1 KB of buf xors (four 32-bit words) to `match` (others
    untouched)."""
    nbytes = buf.numel() * buf.element_size()
    if hits is None:
        hits = torch.zeros(int(lib().kr_stream_read_pieces(nbytes)), dtype=torch.int32, device=buf.device)
    _check(lib().kr_stream_read(_ptr(buf), nbytes, match & 0xFFFFFFFF, _ptr(hits), _stream(stream)))
    return hits


# ---- names of the reference operator surface (encoder.rs) -------------------------------

def encode_q4_linear(weight: Q4Matrix, input: torch.Tensor, output: torch.Tensor, m: int, n: int, k: int,
                     input_byte_offset: int = 0, stream=None) -> None:
    """encoder.rs:2361-2420: output[m, n] = bf16(input[m, k] @ W^T)."""
    if (n, k) != (weight.n, weight.k):
        raise KrError(KR_E_SHAPE, f"weight is [{weight.n},{weight.k}], call says [{n},{k}]")
    x_ptr = _ptr(input) + input_byte_offset
    _check(lib().kr_q4_linear(weight.desc, x_ptr, m, _ptr(output), _dt_of(output), 0, _stream(stream)))


def encode_q4_linear_accumulate(proj_weight: Q4Matrix, input: torch.Tensor, residual_inout: torch.Tensor,
                                n: int, k: int, input_byte_offset: int = 0, stream=None) -> None:
    """encoder.rs:2497-2536: residual[n] = bf16(f32(residual[n]) + W x)."""
    if (n, k) != (proj_weight.n, proj_weight.k):
        raise KrError(KR_E_SHAPE, f"weight is [{proj_weight.n},{proj_weight.k}], call says [{n},{k}]")
    x_ptr = _ptr(input) + input_byte_offset
    _check(lib().kr_q4_linear(proj_weight.desc, x_ptr, 1, _ptr(residual_inout), _dt_of(residual_inout), 1,
                              _stream(stream)))


def encode_fused_gate_up(gate_weight: Q4Matrix, up_weight: Q4Matrix, input: torch.Tensor,
                         mlp_hidden: torch.Tensor, m: int, k: int, intermediate_size: int,
                         activation: int = ACT_SWIGLU, input_byte_offset: int = 0, stream=None) -> None:
    """encoder.rs:2703-2848: mlp_hidden[m, I] = bf16(act(gate x) * up x)."""
    if gate_weight.k != k or gate_weight.n != intermediate_size:
        raise KrError(KR_E_SHAPE, "gate weight shape does not match k / intermediate_size")
    x_ptr = _ptr(input) + input_byte_offset
    _check(lib().kr_q4_gate_up_act(gate_weight.desc, up_weight.desc, x_ptr, m, _ptr(mlp_hidden),
                                   _dt_of(mlp_hidden), activation, _stream(stream)))


def encode_dense_mlp(gate: Q4Matrix, up: Q4Matrix, down: Q4Matrix, norm_out: torch.Tensor,
                     residual: torch.Tensor, num_tokens: int, hidden_size: int, intermediate_size: int,
                     activation: int = ACT_SWIGLU, workspace: Optional[torch.Tensor] = None, stream=None) -> None:
    """encoder.rs:2851-2906: residual += down(act(gate n) * up n) for the normed input n."""
    if down.n != hidden_size or gate.n != intermediate_size:
        raise KrError(KR_E_SHAPE, "MLP weights do not match hidden/intermediate sizes")
    mlp(gate, up, down, residual, x=norm_out, activation=activation, workspace=workspace, stream=stream)
