"""Writes safetensors files for the loader tests (test infrastructure): the
8-byte little-endian header length, the JSON header, then the data section
(safetensors_loader.rs:59-66 describes the format)."""
import json
import struct

import numpy as np


def write(path, tensors, metadata=None, header_len=None, raw_header=None, extra_data=b""):
    """tensors: {name: (dtype, shape, bytes)} in file order.  header_len / raw_header override the
    computed header length / JSON text (malformed-file tests)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, data) in tensors.items():
        data = bytes(data)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    if metadata is not None:
        header["__metadata__"] = metadata
    text = (raw_header if raw_header is not None else json.dumps(header)).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text) if header_len is None else header_len))
        f.write(text)
        for b in blobs:
            f.write(b)
        f.write(extra_data)


def q4_triplet(name, qw, scales, biases, scale_dtype="BF16"):
    """MLX affine triplet entries: U32 [n, k/8] nibbles, scales/biases [n, k/64] (bf16 or f16 bits)."""
    n = qw.shape[0]
    g = scales.shape[1]
    return {f"{name}.weight": ("U32", qw.shape, np.ascontiguousarray(qw, np.uint32).tobytes()),
            f"{name}.scales": (scale_dtype, (n, g), np.ascontiguousarray(scales, np.uint16).tobytes()),
            f"{name}.biases": (scale_dtype, (n, g), np.ascontiguousarray(biases, np.uint16).tobytes())}
