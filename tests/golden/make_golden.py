"""Writes the golden fixtures under tests/golden/.

reference_kats.json — known answers stated in the reference's own tests, as data:
  * DType sizing 256 el -> 144 B                    crates/kriya-core/src/tensor.rs:474
  * MLX triplet repack bytes                        crates/kriya-core/src/safetensors_loader.rs:419-434
  * split / rejoin values                           crates/kriya-core/src/tensor.rs:506-555
  * adversarial bit patterns + LCG round trip       crates/kriya-backend-metal/tests/challenger_m1_adversarial.rs:67-151
  * constant payload 0.03125 (quantize -> dequant)  crates/kriya-backend-metal/tests/test_shader_compile.rs:93-98
  * constant blocks scale 0x3D00, bias 0, qs 0x11   crates/kriya-backend-metal/tests/test_real_qwen.rs:84-91
  * ramp MSE bound 0.005                            crates/kriya-core/src/quantizer.rs:680-695
  * MoE scan/scatter expectations E in {8,64,256}   crates/kriya-backend-metal/tests/test_shader_compile.rs:2988-3117
    (the expected offsets/scatter are computed by that test's own CPU loop, restated below)

closed_form.npz — the closed-form inputs of the reference's GPU tests (weights
quantized with the oracle quantizer) with the oracle's f32 outputs.  These are
regression vectors of the oracle and the inputs of the GPU parity tests.

Run: python tests/golden/make_golden.py   (needs oracle/libkr_oracle.so)
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def f32(a):
    return np.asarray(a, dtype=np.float32)


def lcg_blocks(count: int):
    """challenger_m1_adversarial.rs:118-138: LCG state 0x123456789ABCDEF0, a=6364136223846793005, c=1."""
    mask = (1 << 64) - 1
    st = 0x123456789ABCDEF0
    blocks = []
    for _ in range(count):
        qs = []
        for _ in range(32):
            st = (st * 6364136223846793005 + 1) & mask
            qs.append((st >> 33) & 0xFF)
        st = (st * 6364136223846793005 + 1) & mask
        scale = (st >> 16) & 0xFFFF
        st = (st * 6364136223846793005 + 1) & mask
        bias = (st >> 16) & 0xFFFF
        blocks.append([scale & 0xFF, scale >> 8, bias & 0xFF, bias >> 8] + qs)
    return blocks


def moe_scan_expectation(E: int, T: int = 8, K: int = 4):
    """test_shader_compile.rs:3004-3033."""
    counts = [0] * E
    experts, slots = [], []
    for tok in range(T):
        for k in range(K):
            e = (tok * 7 + k * 13 + 3) % E
            experts.append(e)
            slots.append(counts[e])
            counts[e] += 1
    offsets, run = [], 0
    for e in range(E):
        offsets.append(run)
        run += counts[e]
    offsets.append(run)
    scatter = [0] * (T * K)
    for i, (e, s) in enumerate(zip(experts, slots)):
        scatter[offsets[e] + s] = i
    return {"E": E, "T": T, "K": K, "experts": experts, "slots": slots, "offsets": offsets, "scatter": scatter}


def kats() -> dict:
    return {
        "dtype_sizing": {"elements": 256, "bytes": 144},
        "mlx_repack": {
            "weight_nibbles": [0xAB] * 64,
            "scales": [0x3F80, 0x4000],
            "biases": [0x0000, 0x3C00],
            "expect_scale": [0x3F80, 0x4000],
            "expect_bias": [0x0000, 0x3C00],
            "expect_qs0": [0xAB, 0xAB],
            # dequant by hand: low nibble 0xB = 11 (even element), high 0xA = 10 (odd);
            # block 0: s = 1.0, b = 0 -> 11, 10; block 1: s = 2.0, b = 2^-7 -> 22.0078125, 20.0078125
            "expect_dequant_first_pair": [[11.0, 10.0], [22.0078125, 20.0078125]],
        },
        "split_rejoin": {
            "blocks": [{"scale": i * 10, "bias": i * 5, "qs": [i] * 32} for i in range(8)],
            "expect_qs3_0": 3, "expect_sb3": [30, 15], "expect_single4": [4, 40],
        },
        "adversarial_patterns": [
            {"scale": 0x0000, "bias": 0x0000, "qs": 0x00},
            {"scale": 0xFFFF, "bias": 0xFFFF, "qs": 0xFF},
            {"scale": 0x7F80, "bias": 0xFF80, "qs": 0x5A},
            {"scale": 0x0001, "bias": 0x8000, "qs": 0xA5},
        ],
        "lcg_blocks_1000": lcg_blocks(1000),
        "constant_payload": {"value": 0.03125, "elements": 64 * 64},
        "constant_blocks": {"scale": 0x3D00, "bias": 0x0000, "qs": 0x11, "w": 0.03125},
        "ramp_mse": {"n": 128, "start": -64.0, "step": 0.05, "mse_below": 0.005},
        "moe_scan_scatter": [moe_scan_expectation(E) for E in (8, 64, 256)],
    }


def quantized(n: int, k: int, fn):
    idx = np.arange(n * k)
    w = f32(fn(idx))
    blocks = oracle.quantize_q4_g64(w)
    return oracle.blocks36_to_planar(blocks, n, k), blocks


def closed_form() -> dict:
    out = {}

    def gemv_case(name, n, k, wfn, xfn):
        w, blocks = quantized(n, k, wfn)
        x = oracle.f32_to_bf16(f32(xfn(np.arange(k))))
        out[f"{name}_qw"], out[f"{name}_sc"], out[f"{name}_bi"] = w.qw, w.scales, w.biases
        out[f"{name}_blocks"] = blocks
        out[f"{name}_x"] = x
        out[f"{name}_y"] = oracle.q4_matmul(w, x)[0]

    # test_shader_compile.rs:577-586, 654-662, 849-857
    gemv_case("gemv_5x64", 5, 64, lambda i: ((i % 37) - 18.0) * 0.03125, lambda i: ((i % 11) - 5.0) * 0.125)
    gemv_case("gemv_7x128", 7, 128, lambda i: ((i % 37) - 18.0) * 0.03125, lambda i: ((i % 11) - 5.0) * 0.125)
    gemv_case("gemv_19x128", 19, 128, lambda i: ((i % 41) - 20.0) * 0.03125, lambda i: ((i % 13) - 6.0) * 0.125)

    def swiglu_case(name, inter, k, gfn, ufn, xfn):
        g, _ = quantized(inter, k, gfn)
        u, _ = quantized(inter, k, ufn)
        x = oracle.f32_to_bf16(f32(xfn(np.arange(k))))
        for tag, w in (("g", g), ("u", u)):
            out[f"{name}_{tag}qw"], out[f"{name}_{tag}sc"], out[f"{name}_{tag}bi"] = w.qw, w.scales, w.biases
        out[f"{name}_x"] = x
        out[f"{name}_a"] = oracle.q4_gate_up_act(g, u, x)[0]

    # test_shader_compile.rs:732-748, 927-943
    swiglu_case("swiglu_9x128", 9, 128, lambda i: ((i % 29) - 14.0) * 0.03125,
                lambda i: ((i % 31) - 15.0) * 0.03125, lambda i: ((i % 13) - 6.0) * 0.1)
    swiglu_case("swiglu_11x128", 11, 128, lambda i: ((i % 33) - 16.0) * 0.03125,
                lambda i: ((i % 37) - 18.0) * 0.03125, lambda i: ((i % 17) - 8.0) * 0.1)

    # test_shader_compile.rs:1603-1616: M=64, N=64, K=128
    w, _ = quantized(64, 128, lambda i: ((i % 23) - 11.0) * 0.05)
    x = oracle.f32_to_bf16(f32(((np.arange(64 * 128) % 19) - 9.0) * 0.04)).reshape(64, 128)
    out["gemm_64x64x128_qw"], out["gemm_64x64x128_sc"], out["gemm_64x64x128_bi"] = w.qw, w.scales, w.biases
    out["gemm_64x64x128_x"] = x
    out["gemm_64x64x128_y"] = oracle.q4_matmul(w, x)

    # test_shader_compile.rs:2513-2530: N = K = 256 blocks with fixed scale/bias and a byte pattern
    nb = 256 * 4
    blocks = np.zeros((nb, 36), np.uint8)
    s, b = oracle.f32_to_bf16(f32([0.05]))[0], oracle.f32_to_bf16(f32([-0.4]))[0]
    blocks[:, 0], blocks[:, 1] = s & 0xFF, s >> 8
    blocks[:, 2], blocks[:, 3] = b & 0xFF, b >> 8
    bi_, byte_i = np.meshgrid(np.arange(nb), np.arange(32), indexing="ij")
    blocks[:, 4:] = ((bi_ * 31 + byte_i * 7) % 256).astype(np.uint8)
    w = oracle.blocks36_to_planar(blocks, 256, 256)
    x = oracle.f32_to_bf16(f32(((np.arange(256) % 13) - 6.0) * 0.1))
    out["persist_256_qw"], out["persist_256_sc"], out["persist_256_bi"] = w.qw, w.scales, w.biases
    out["persist_256_x"] = x
    out["persist_256_y"] = oracle.q4_matmul(w, x)[0]
    return out


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(kats(), f, separators=(",", ":"))
    np.savez_compressed(os.path.join(HERE, "closed_form.npz"), **closed_form())
    print("wrote reference_kats.json, closed_form.npz")


if __name__ == "__main__":
    main()
