"""The reference's own real-dimension and invariant tests of this path, at their shapes and with
their inputs, through the C ABI:

  * Llama-3.2-3B decode GEMV, 3072 x 3072 (real_world_validation.rs:43-152): weights
    ((i * 1e-4 - 0.5) * 0.01), input ((i * 2e-4 - 0.3) * 0.01), quantized by the reference's
    quantizer (the oracle's port of quantize_f32_to_q4_group64), bound to the device through the
    36-byte block conversion;
  * prefill GEMM, M = 16, K = 3072, N = 3072 (:154-289): inputs ((i * 1e-4 - 0.5) * 0.01),
    weights ((i * 5e-5 - 0.25) * 0.01), and again at M = 64 and 512 on the prefill kernel;
  * fused SwiGLU decode invariant 4 (challenger_m1_2_resilience.rs:357-455): constant blocks
    scale 0x3D00, bias 0, qs 0x22 (every nibble 2, w = 0.0625), x = 0.5, k = 64, 64 features:
    every output is silu(2) * 2 exactly up to bf16 rounding;
  * batched versus token-by-token (real_world_validation.rs:707-760 compares forward_prefill_batch
    with token-at-a-time decode): a batched launch equals, row for row, m = 1 launches of the same
    rows, within the bar.

Bars: the reference's own (|d| > 0.05 and rel > 0.05 fails for the GEMV; a mismatch rate below 1 %
for the prefill GEMM) and the parity bar max |gpu - oracle| <= 1e-2 RMS(oracle), bf16 outputs
the RNE of a value within it."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)


def reference_blocks(n, k, scale, offset):
    """quantize_f32_to_q4_group64 of ((i * scale - offset) * 0.01), i over the row-major [n, k] matrix."""
    i = np.arange(n * k, dtype=np.float64)
    w = ((i * scale - offset) * 0.01).astype(np.float32)
    return O.quantize_q4_g64(w)


def on_device(kq, blocks, n, k):
    return kq.Q4Matrix.from_blocks36(torch.from_numpy(np.ascontiguousarray(blocks)).cuda(), n, k)


def reference_tolerance(gpu, cpu, abs_tol, rel_tol):
    diff = np.abs(gpu - cpu)
    rel = np.where(np.abs(cpu) > 1e-6, diff / np.maximum(np.abs(cpu), 1e-30), diff)
    return (diff > abs_tol) & (rel > rel_tol)


def test_llama3b_decode_gemv_3072(kq):
    h = q_dim = 3072
    case(f"Llama-3.2-3B decode GEMV {q_dim} x {h} from the reference's quantizer")
    blocks = reference_blocks(q_dim, h, 1e-4, 0.5)
    w = O.blocks36_to_planar(blocks, q_dim, h)
    x = O.f32_to_bf16((np.arange(h, dtype=np.float64) * 2e-4 - 0.3) * 0.01)
    want = O.q4_matmul(w, x)[0]
    y = kq.q4_linear(on_device(kq, blocks, q_dim, h), dev_bf16(x), out_dtype=kq.DTYPE_BF16)
    got_bits = host_bits(y)[0]
    got = O.bf16_to_f32(got_bits)
    assert not reference_tolerance(got, want, 0.05, 0.05).any()
    assert_bf16_rounded_close(got_bits, want, rms(want), what="llama3b gemv")
    y32 = kq.q4_linear(on_device(kq, blocks, q_dim, h), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
    assert_rms_close(y32, want, what="llama3b gemv f32")


@pytest.mark.parametrize("m", [16, 64, 512])
def test_prefill_gemm_3072(kq, m):
    k = n = 3072
    case(f"prefill GEMM m={m} k={k} n={n} with the reference's inputs")
    blocks = reference_blocks(n, k, 5e-5, 0.25)
    w = O.blocks36_to_planar(blocks, n, k)
    i = np.arange(16 * k, dtype=np.float64)
    x16 = O.f32_to_bf16(((i * 1e-4 - 0.5) * 0.01).reshape(16, k))
    x = np.tile(x16, (m // 16, 1)) if m > 16 else x16  # the reference's 16 rows, repeated
    want = O.q4_matmul(w, x)
    wd = on_device(kq, blocks, n, k)
    got_bits = host_bits(kq.q4_linear(wd, dev_bf16(x), out_dtype=kq.DTYPE_BF16))
    got = O.bf16_to_f32(got_bits)
    mism = reference_tolerance(got, want, 0.05, 0.1)
    assert mism.mean() * 100.0 < 1.0
    assert_bf16_rounded_close(got_bits, want, rms(want), what=f"prefill m={m}")
    y32 = kq.q4_linear(wd, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y32, want, what=f"prefill m={m} f32")


def test_swiglu_invariant_constant_blocks(kq):
    k = inter = 64
    case("fused SwiGLU decode with constant blocks (scale 0x3D00, bias 0, qs 0x22), x = 0.5")
    blk = np.zeros(36, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(0x3D00).tobytes(), np.uint8)  # scale bf16 (little-endian)
    blk[2:4] = 0  # bias
    blk[4:36] = 0x22
    blocks = np.tile(blk, (inter * (k // 64), 1))
    gate = on_device(kq, blocks, inter, k)
    up = on_device(kq, blocks, inter, k)
    x = O.f32_to_bf16(np.full((1, k), 0.5, np.float32))
    out = kq.gate_up_act(gate, up, dev_bf16(x), out_dtype=kq.DTYPE_BF16)
    got = O.bf16_to_f32(host_bits(out))[0]
    assert np.all(np.isfinite(got)) and np.all(got > 0.0)  # the reference's assertions
    g = 64 * (2 * 0.03125) * 0.5  # = 2.0 exactly
    exact = g / (1.0 + math.exp(-g)) * g
    assert np.all(np.abs(got - exact) <= abs(exact) * 2.0 ** -8)
    # the same with 16 tokens (few-token kernel)
    x16 = O.f32_to_bf16(np.full((16, k), 0.5, np.float32))
    out16 = O.bf16_to_f32(host_bits(kq.gate_up_act(gate, up, dev_bf16(x16), out_dtype=kq.DTYPE_BF16)))
    assert np.all(np.abs(out16 - exact) <= abs(exact) * 2.0 ** -8)


@pytest.mark.parametrize("m", [4, 16, 48, 96])
def test_batched_matches_token_by_token(kq, m):
    from kriya_q4 import synth
    n, k = 1024, 2048
    case(f"batched launch m={m} vs m = 1 launches of the same rows, n={n} k={k}")
    wq = synth.q4_weight(n, k, 8800 + m)
    wd = q4_dev(kq, wq)
    x = synth.bf16_normal((m, k), 8801 + m)
    batched = kq.q4_linear(wd, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    rows = np.stack([kq.q4_linear(wd, dev_bf16(x[i:i + 1]), out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
                     for i in range(m)])
    assert_rms_close(batched, rows, what=f"batched vs token-by-token m={m}")
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    assert_rms_close(batched, want, what=f"batched m={m} vs oracle")
    # the MLP step too: batched against token-at-a-time (the residual h is updated in place)
    H, I = 512, 1024
    g, u, d = synth.q4_weight(I, H, 8810), synth.q4_weight(I, H, 8811), synth.q4_weight(H, I, 8812)
    gd, ud, dd = q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d)
    h0 = synth.bf16_normal((m, H), 8813 + m)
    hb = dev_bf16(h0)
    kq.mlp(gd, ud, dd, hb, workspace=kq.mlp_workspace(m, H, I))
    ws1 = kq.mlp_workspace(1, H, I)
    ht = []
    for i in range(m):
        hi = dev_bf16(h0[i:i + 1])
        kq.mlp(gd, ud, dd, hi, workspace=ws1)
        ht.append(O.bf16_to_f32(host_bits(hi))[0])
    hb_f = O.bf16_to_f32(host_bits(hb)).astype(np.float64)
    ht_f = np.stack(ht).astype(np.float64)
    ref = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    want = O.bf16_to_f32(h0).astype(np.float64) + ref
    # both are bf16(h + mlp): each within its own rounding plus the bar of the oracle, and so within
    # twice that of each other
    bound_b = np.abs(hb_f) * 2.0 ** -8 + 1e-2 * rms(ref)
    bound_t = np.abs(ht_f) * 2.0 ** -8 + 1e-2 * rms(ref)
    assert np.all(np.abs(hb_f - want) <= bound_b)
    assert np.all(np.abs(ht_f - want) <= bound_t)
    assert np.all(np.abs(hb_f - ht_f) <= bound_b + bound_t)
