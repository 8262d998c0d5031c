"""Checkpoint archives (include/kriya_loader.h) from Python: safetensors files or
sharded directories, mapped by the C++ reader in libkriya_q4.so, and their Q4
projections loaded into device-resident ``Q4Matrix`` planar triplets.

Mirrors kriya-core's ``ShardedCheckpointLoader`` (crates/kriya-core/src/
safetensors_loader.rs:122-208) and kriya-backend-metal's bind/validate step
(crates/kriya-backend-metal/src/encoder.rs:452-591, 651-703).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from . import KrError, Q4Matrix, _stream, lib

KR_E_IO, KR_E_FORMAT, KR_E_MISSING = -7, -8, -9
ST_DTYPES = ["F32", "F16", "BF16", "F8_E4M3", "Q4_G64", "Q2_G128", "Q3_G64", "U32", "U8", "I32", "I8"]
_NP = {"F32": np.float32, "F16": np.uint16, "BF16": np.uint16, "U32": np.uint32, "U8": np.uint8, "I32": np.int32,
       "I8": np.int8, "F8_E4M3": np.uint8, "Q4_G64": np.uint8, "Q2_G128": np.uint8, "Q3_G64": np.uint8}


class kr_tensor_info(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8),
                ("byte_len", ctypes.c_uint64), ("data", ctypes.c_void_p), ("shard", ctypes.c_char_p)]


class kr_dense_model_desc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_uint32), ("intermediate", ctypes.c_uint32), ("layers", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("q_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("qkv_bias", ctypes.c_int), ("tie_word_embeddings", ctypes.c_int)]


_declared = False


def _L():
    global _declared
    L = lib()
    if not _declared:
        vp, u32, u64, i32, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_size_t
        sig = {
            "kr_archive_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            "kr_archive_close": (None, [vp]),
            "kr_archive_tensor_count": (sz, [vp]),
            "kr_archive_tensor_name": (ctypes.c_char_p, [vp, sz]),
            "kr_archive_tensor": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(kr_tensor_info)]),
            "kr_archive_check_q4": (i32, [vp, ctypes.c_char_p, u32, u32, ctypes.POINTER(ctypes.c_int)]),
            "kr_archive_q4_staging_bytes": (i32, [vp, ctypes.c_char_p, u32, u32, ctypes.POINTER(sz)]),
            "kr_archive_load_q4": (i32, [vp, ctypes.c_char_p, u32, u32, vp, vp, vp, vp, sz, vp]),
            "kr_archive_load_bf16": (i32, [vp, ctypes.c_char_p, u64, vp, vp]),
            "kr_checkpoint_validate_dense": (i32, [vp, ctypes.POINTER(kr_dense_model_desc)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise KrError(rc, _L().kr_last_error().decode())


class Archive:
    """A mapped checkpoint: a .safetensors file, or a directory with model.safetensors.index.json
    (sharded) or model.safetensors (ShardedCheckpointLoader::open)."""

    def __init__(self, path: str):
        self._h = ctypes.c_void_p()
        _check(_L().kr_archive_open(str(path).encode(), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            _L().kr_archive_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        L = _L()
        return [L.kr_archive_tensor_name(self._h, i).decode() for i in range(L.kr_archive_tensor_count(self._h))]

    def info(self, name: str) -> dict:
        ti = kr_tensor_info()
        _check(_L().kr_archive_tensor(self._h, name.encode(), ctypes.byref(ti)))
        return {"dtype": ST_DTYPES[ti.dtype], "shape": [int(ti.shape[i]) for i in range(ti.ndim)],
                "byte_len": int(ti.byte_len), "data": ti.data, "shard": ti.shard.decode()}

    def host_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only view of the mapping (valid while the archive is open)."""
        i = self.info(name)
        buf = (ctypes.c_uint8 * i["byte_len"]).from_address(i["data"]) if i["byte_len"] else b""
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def check_q4(self, prefix: str, n: int, k: int) -> int:
        """1: a Q4_G64 tensor (36-byte blocks); 2: an MLX .weight/.scales/.biases triplet."""
        p = ctypes.c_int()
        _check(_L().kr_archive_check_q4(self._h, prefix.encode(), n, k, ctypes.byref(p)))
        return p.value

    def load_q4(self, prefix: str, n: int, k: int, device="cuda", stream=None) -> Q4Matrix:
        """bind_q4_buffer (encoder.rs:651-703): the projection as a planar Q4Matrix on the device."""
        w = Q4Matrix.empty(n, k, device=device)
        need = ctypes.c_size_t()
        _check(_L().kr_archive_q4_staging_bytes(self._h, prefix.encode(), n, k, ctypes.byref(need)))
        staging: Optional[torch.Tensor] = None
        if need.value:
            staging = torch.empty(need.value, dtype=torch.uint8, device=device)
        _check(_L().kr_archive_load_q4(self._h, prefix.encode(), n, k, w.qw.data_ptr(), w.scales.data_ptr(),
                                       w.biases.data_ptr(), staging.data_ptr() if staging is not None else None,
                                       need.value, _stream(stream)))
        return w

    def load_bf16(self, name: str, length: int, device="cuda", stream=None) -> torch.Tensor:
        out = torch.empty(length, dtype=torch.bfloat16, device=device)
        _check(_L().kr_archive_load_bf16(self._h, name.encode(), length, out.data_ptr(), _stream(stream)))
        return out

    def validate_dense(self, hidden, intermediate, layers, vocab, q_heads, kv_heads, head_dim, qkv_bias=True,
                       tie_word_embeddings=True) -> None:
        """validate_production_checkpoint (encoder.rs:452-591) for a dense GQA decoder; raises on failure."""
        d = kr_dense_model_desc(hidden, intermediate, layers, vocab, q_heads, kv_heads, head_dim, int(qkv_bias),
                                int(tie_word_embeddings))
        _check(_L().kr_checkpoint_validate_dense(self._h, ctypes.byref(d)))
