"""Pins the CPU oracle (oracle/kr_oracle.c) before it is trusted as the checker.

What pins each oracle function (beyond restating it):
  f32_to_bf16       torch's float32->bfloat16 (RNE, independent implementation) on 2^24 strided
                    patterns + every exponent; hand-worked wrap-around cases for NaN inputs
  f16_to_f32        numpy float16->float32 bit patterns, all 65536 inputs
  half_to_bf16      composition of the two pinned conversions
  quantize_q4_g64   reference KATs: ramp MSE < 0.005, constant 0.03125; round-half-away-from-zero
                    case; error <= scale/2 property; reference length error
  dequant           reference KATs (MLX repack bytes, constant blocks 0x3D00/0x11); float64
                    q*s+b (exact) rounded once to float32 == fmaf on random blocks
  layouts           reference KATs (repack, split/rejoin, adversarial patterns, 1000 LCG blocks)
                    plus planar <-> 36 B round trips
  q4_matmul         one-hot inputs select a dequantized column exactly; float64 numpy matmul
                    within the f32 summation bound; constant-weight closed form y = 0.03125 * sum(x)
  activation        numpy float64 silu / tanh-gelu / relu
  gate_up / mlp     numpy float64 composition of pinned pieces
  moe_route         numpy float64 softmax + stable argsort (ties to the lower id) + renorm
  moe_scan_scatter  the reference test's own expectations for E in {8, 64, 256}
  moe_experts       numpy float64 composition of pinned pieces
"""
import json
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def test_f32_to_bf16_matches_torch_rne():
    import torch

    rng = np.random.default_rng(0)
    pats = np.concatenate([
        np.arange(0, 1 << 32, 1 << 8, dtype=np.uint64)[: 1 << 24].astype(np.uint32),
        rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32),
        (np.arange(256, dtype=np.uint32) << 23) | 0x8000,  # exact ties at every exponent
        (np.arange(256, dtype=np.uint32) << 23) | 0x18000,
    ])
    f = pats.view(np.float32)
    finite = np.isfinite(f)
    ours = O.f32_to_bf16(f[finite])
    ref = torch.from_numpy(f[finite]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f32_to_bf16_nan_wraps_like_reference():
    # quantizer.rs:19-24 adds 0x7FFF + lsb in wrapping u32 arithmetic and shifts.
    cases = {0x7F800001: 0x7F80, 0x7FC00000: 0x7FC0, 0xFFFFFFFF: 0x0000, 0x7FFFFFFF: 0x8000, 0xFF800001: 0xFF80}
    for bits, want in cases.items():
        got = int(O.f32_to_bf16(np.array([bits], np.uint32).view(np.float32))[0])
        assert got == want, hex(bits)


def test_f16_to_f32_all_patterns_match_numpy():
    h = np.arange(1 << 16, dtype=np.uint16)
    ours = O.f16_to_f32(h).view(np.uint32)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(ours, ref)


def test_half_to_bf16_composition():
    for raw in (0x3C00, 0x0001, 0x8001, 0x7BFF, 0x7C00, 0xFC00, 0x3555, 0x0400):
        f = np.array([raw], np.uint16).view(np.float16).astype(np.float32)
        assert O.half_to_bf16(raw, True) == int(O.f32_to_bf16(f)[0])
        assert O.half_to_bf16(raw, False) == raw


def test_quantizer_ramp_mse_kat():
    k = KATS["ramp_mse"]
    w = (np.arange(k["n"], dtype=np.float32) + np.float32(k["start"])) * np.float32(k["step"])
    blocks = O.quantize_q4_g64(w)
    assert blocks.shape == (2, 36)
    mse = float(np.mean((w - O.dequant_blocks36(blocks)) ** 2))
    assert mse < k["mse_below"]


def test_quantizer_constant_payload_kat():
    k = KATS["constant_payload"]
    w = np.full(k["elements"], k["value"], np.float32)
    deq = O.dequant_blocks36(O.quantize_q4_g64(w))
    assert np.all(deq == np.float32(k["value"]))


def test_quantizer_rounds_half_away_from_zero():
    # min 0 and max 15 give scale exactly 1.0, bias 0: 2.5 -> 3 (Rust f32::round), not 2 (ties-to-even).
    w = np.zeros(64, np.float32)
    w[1] = 15.0
    w[2], w[3] = 2.5, 4.5
    q = O.quantize_q4_g64(w)[0]
    assert (q[4 + 1] & 0x0F) == 3 and (q[4 + 1] >> 4) == 5


def test_quantizer_error_bound_and_length_error():
    rng = np.random.default_rng(1)
    w = rng.standard_normal(64 * 50).astype(np.float32)
    blocks = O.quantize_q4_g64(w)
    deq = O.dequant_blocks36(blocks).reshape(50, 64)
    s = O.bf16_to_f32(blocks[:, 0].astype(np.uint16) | (blocks[:, 1].astype(np.uint16) << 8))
    b = O.bf16_to_f32(blocks[:, 2].astype(np.uint16) | (blocks[:, 3].astype(np.uint16) << 8))
    wr = w.reshape(50, 64)
    inside = (wr >= b[:, None]) & (wr <= (b + 15 * s)[:, None])
    err = np.abs(wr - deq)
    assert np.all(err[inside] <= (0.5 * s[:, None] + 1e-6 * np.abs(wr))[inside])
    with pytest.raises(ValueError):
        O.quantize_q4_g64(np.zeros(65, np.float32))


def _blocks_from_kat(entries):
    out = np.zeros((len(entries), 36), np.uint8)
    for i, e in enumerate(entries):
        out[i, 0], out[i, 1] = e["scale"] & 0xFF, e["scale"] >> 8
        out[i, 2], out[i, 3] = e["bias"] & 0xFF, e["bias"] >> 8
        out[i, 4:] = e["qs"] if isinstance(e["qs"], list) else [e["qs"]] * 32
    return out


def test_mlx_repack_kat_and_dequant():
    k = KATS["mlx_repack"]
    blocks = O.mlx_pack_blocks36(np.array(k["weight_nibbles"], np.uint8), np.array(k["scales"], np.uint16), False,
                                 np.array(k["biases"], np.uint16), False)
    assert blocks.shape == (2, 36)
    for i in range(2):
        assert int(blocks[i, 0]) | int(blocks[i, 1]) << 8 == k["expect_scale"][i]
        assert int(blocks[i, 2]) | int(blocks[i, 3]) << 8 == k["expect_bias"][i]
        assert blocks[i, 4] == k["expect_qs0"][i]
    deq = O.dequant_blocks36(blocks).reshape(2, 64)
    for i in range(2):
        assert deq[i, 0] == np.float32(k["expect_dequant_first_pair"][i][0])
        assert deq[i, 1] == np.float32(k["expect_dequant_first_pair"][i][1])
    with pytest.raises(ValueError):
        O.mlx_pack_blocks36(np.zeros(33, np.uint8), np.zeros(1, np.uint16), False, np.zeros(1, np.uint16), False)
    with pytest.raises(ValueError):
        O.mlx_pack_blocks36(np.zeros(64, np.uint8), np.zeros(1, np.uint16), False, np.zeros(2, np.uint16), False)


def test_mlx_repack_f16_scales_convert():
    wb = np.full(32, 0x21, np.uint8)
    s16 = np.array([0x3555], np.uint16)  # f16 0.33325..., not exact in bf16
    blocks = O.mlx_pack_blocks36(wb, s16, True, np.array([0xBC00], np.uint16), True)
    s = int(blocks[0, 0]) | int(blocks[0, 1]) << 8
    assert s == O.half_to_bf16(0x3555, True) and s != 0x3555
    assert (int(blocks[0, 2]) | int(blocks[0, 3]) << 8) == 0xBF80  # f16 -1.0 -> bf16 -1.0


def test_split_rejoin_kats():
    k = KATS["split_rejoin"]
    blocks = _blocks_from_kat(k["blocks"])
    qs, sb = O.split_blocks36(blocks)
    assert qs[3, 0] == k["expect_qs3_0"] and list(sb[3]) == k["expect_sb3"]
    assert qs[4, 0] == k["expect_single4"][0] and sb[4, 0] == k["expect_single4"][1]
    assert np.array_equal(O.join_blocks36(qs, sb), blocks)
    pats = _blocks_from_kat(KATS["adversarial_patterns"])
    assert np.array_equal(O.join_blocks36(*O.split_blocks36(pats)), pats)
    lcg = np.array(KATS["lcg_blocks_1000"], np.uint8)
    assert np.array_equal(O.join_blocks36(*O.split_blocks36(lcg)), lcg)
    empty = np.zeros((0, 36), np.uint8)
    assert O.join_blocks36(*O.split_blocks36(empty)).shape == (0, 36)


def test_planar_blocks_round_trip_and_nibble_order():
    lcg = np.array(KATS["lcg_blocks_1000"], np.uint8)  # 1000 blocks = 8 rows x 125 groups
    w = O.blocks36_to_planar(lcg, 8, 125 * 64)
    assert np.array_equal(O.planar_to_blocks36(w), lcg)
    # byte i of a block = element 2i (low nibble) and 2i+1 (high): qs[0] of block (0,0) is word 0 byte 0
    assert (int(w.qw[0, 0]) & 0xFF) == lcg[0, 4]
    assert sizing_bytes(256) == KATS["dtype_sizing"]["bytes"]


def sizing_bytes(elements: int) -> int:
    return -(-elements // 64) * 36  # DType::Q4Group64 block sizing (tensor.rs:75, 88)


def test_dequant_matches_float64_exact_rounding():
    rng = np.random.default_rng(2)
    n, k = 16, 256
    qw = rng.integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_bf16(rng.uniform(1e-3, 0.1, size=(n, k // 64)).astype(np.float32))
    bi = O.f32_to_bf16(rng.uniform(-1, 1, size=(n, k // 64)).astype(np.float32))
    deq = O.dequant_planar(O.Q4Planar(qw, sc, bi))
    q = ((qw[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(n, k).astype(np.float64)
    s = np.repeat(O.bf16_to_f32(sc).astype(np.float64), 64, axis=1)
    b = np.repeat(O.bf16_to_f32(bi).astype(np.float64), 64, axis=1)
    assert np.array_equal(deq, (q * s + b).astype(np.float32))


def test_dequant_constant_blocks_kat():
    k = KATS["constant_blocks"]
    blocks = _blocks_from_kat([{"scale": k["scale"], "bias": k["bias"], "qs": k["qs"]}] * 4)
    assert np.all(O.dequant_blocks36(blocks) == np.float32(k["w"]))


def _rand_w(n, k, seed):
    from kriya_q4 import synth
    return O.Q4Planar(*synth.q4_weight(n, k, seed))


def test_matmul_one_hot_selects_columns():
    w = _rand_w(24, 192, 3)
    deq = O.dequant_planar(w)
    for col in (0, 1, 7, 63, 64, 191):
        x = np.zeros(192, np.uint16)
        x[col] = 0x3F80  # 1.0
        assert np.array_equal(O.q4_matmul(w, x)[0], deq[:, col])


def test_matmul_matches_float64_within_sum_bound():
    from kriya_q4 import synth
    w = _rand_w(33, 640, 4)
    x = synth.bf16_normal((3, 640), 5)
    y = O.q4_matmul(w, x)
    deq = O.dequant_planar(w).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    ref = xf @ deq.T
    bound = 640 * 2.0 ** -24 * (np.abs(xf) @ np.abs(deq).T) * 1.01
    assert np.all(np.abs(y - ref) <= bound)
    assert np.allclose(O.q4_matmul_f64(w, x), ref, rtol=1e-12, atol=1e-12)


def test_matmul_constant_weight_closed_form():
    k = KATS["constant_blocks"]
    n, kk = 3, 128
    blocks = _blocks_from_kat([{"scale": k["scale"], "bias": k["bias"], "qs": k["qs"]}] * (n * kk // 64))
    w = O.blocks36_to_planar(blocks, n, kk)
    x = O.f32_to_bf16(np.linspace(-2, 2, kk).astype(np.float32))
    y = O.q4_matmul_f64(w, x)[0]
    assert np.allclose(y, 0.03125 * O.bf16_to_f32(x).astype(np.float64).sum(), rtol=0, atol=1e-12)


def test_activation_against_float64():
    g = np.linspace(-20, 20, 4001).astype(np.float32)
    gd = g.astype(np.float64)
    silu = gd / (1 + np.exp(-gd))
    gelu = 0.5 * gd * (1 + np.tanh(0.7978845608 * (gd + 0.044715 * gd ** 3)))
    # f32 evaluation error scales with |g| where 1 + exp(-g) or 1 + tanh(.) cancels
    for v, ref, tol in ((0, silu, 1e-6), (1, gelu, 1e-6), (2, np.maximum(gd, 0), 0)):
        ours = np.array([O.activation(float(t), v) for t in g], np.float64)
        assert np.all(np.abs(ours - ref) <= tol * (np.abs(ref) + np.abs(gd))), v


def _f64_matmul(w, xf):
    return xf @ O.dequant_planar(w).astype(np.float64).T


def test_gate_up_and_mlp_against_float64():
    from kriya_q4 import synth
    h, inter = 128, 192
    g, u, d = _rand_w(inter, h, 6), _rand_w(inter, h, 7), _rand_w(h, inter, 8)
    x = synth.bf16_normal((2, h), 9)
    xf = O.bf16_to_f32(x).astype(np.float64)
    gg, uu = _f64_matmul(g, xf), _f64_matmul(u, xf)
    a_ref = gg / (1 + np.exp(-gg)) * uu
    a = O.q4_gate_up_act(g, u, x)
    assert np.allclose(a, a_ref, rtol=1e-4, atol=1e-4 * np.abs(a_ref).max())
    y = O.q4_mlp(g, u, d, x, bf16_intermediate=False)
    y_ref = _f64_matmul(d, a_ref)
    assert np.allclose(y, y_ref, rtol=1e-4, atol=1e-4 * np.abs(y_ref).max())
    yb = O.q4_mlp(g, u, d, x, bf16_intermediate=True)
    y_ref_b = _f64_matmul(d, O.bf16_to_f32(O.f32_to_bf16(a)).astype(np.float64))
    assert np.allclose(yb, y_ref_b, rtol=1e-4, atol=1e-4 * np.abs(y_ref_b).max())


def test_moe_route_against_numpy():
    from kriya_q4 import synth
    T, E, K = 64, 60, 4
    logits = synth.f32_normal((T, E), 10)
    logits[3, 5] = logits[3, 9] = 9.0  # a tie: expert 5 must come first
    experts, weights, counts, offsets, sorted_assign = O.moe_route(logits, K, True)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    top = np.argsort(-p, axis=1, kind="stable")[:, :K]
    assert np.array_equal(experts, top)
    assert experts[3, 0] == 5 and experts[3, 1] == 9
    pw = np.take_along_axis(p, top, 1)
    assert np.allclose(weights, pw / pw.sum(1, keepdims=True), rtol=1e-5)
    assert np.array_equal(counts, np.bincount(experts.ravel(), minlength=E))
    assert offsets[-1] == T * K and np.all(np.diff(offsets.astype(np.int64)) == counts)
    flat = experts.ravel()
    assert np.array_equal(sorted_assign, np.argsort(flat, kind="stable"))
    ew, *_ = O.moe_route(logits, K, False)
    _, w_un, *_ = O.moe_route(logits, K, False)
    assert np.allclose(w_un, pw, rtol=1e-5)
    with pytest.raises(ValueError):
        O.moe_route(logits, 61, True)


def test_moe_scan_scatter_reference_expectations():
    for case in KATS["moe_scan_scatter"]:
        counts, offsets, scatter = O.moe_scan_scatter(np.array(case["experts"], np.uint32), case["E"])
        assert list(offsets) == case["offsets"]
        assert list(scatter) == case["scatter"]


def test_moe_experts_against_float64():
    from kriya_q4 import synth
    E, H, I, T, K = 6, 128, 128, 5, 2
    g, u, d = _rand_w(E * I, H, 11), _rand_w(E * I, H, 12), _rand_w(E * H, I, 13)
    x = synth.bf16_normal((T, H), 14)
    logits = synth.f32_normal((T, E), 15)
    experts, weights, *_ = O.moe_route(logits, K, True)
    y = O.moe_experts(g, u, d, E, x, experts, weights)
    xf = O.bf16_to_f32(x).astype(np.float64)
    ref = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            e = int(experts[t, k])
            gg = _f64_matmul(g.rows(e * I, (e + 1) * I), xf[t:t + 1])
            uu = _f64_matmul(u.rows(e * I, (e + 1) * I), xf[t:t + 1])
            a = O.bf16_to_f32(O.f32_to_bf16((gg / (1 + np.exp(-gg)) * uu).astype(np.float32))).astype(np.float64)
            ref[t] += weights[t, k] * _f64_matmul(d.rows(e * H, (e + 1) * H), a)[0]
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_closed_form_fixtures_regress():
    z = np.load(os.path.join(HERE, "golden", "closed_form.npz"))
    for name in ("gemv_5x64", "gemv_7x128", "gemv_19x128", "persist_256"):
        w = O.Q4Planar(z[f"{name}_qw"], z[f"{name}_sc"], z[f"{name}_bi"])
        assert np.array_equal(O.q4_matmul(w, z[f"{name}_x"])[0], z[f"{name}_y"]), name
    # the reference test tolerance against its own f32 expectation (|gpu - cpu| < 0.05) holds trivially here
    w = O.Q4Planar(z["gemm_64x64x128_qw"], z["gemm_64x64x128_sc"], z["gemm_64x64x128_bi"])
    assert np.array_equal(O.q4_matmul(w, z["gemm_64x64x128_x"]), z["gemm_64x64x128_y"])


def test_f32_matmul_on_predequantised_rows_equals_q4_matmul():
    """The CPU baseline's upper-bound variant (dot on weights dequantised beforehand) performs the same
    roundings in the same order as the faithful path, so the results are identical bit for bit."""
    from kriya_q4 import synth
    w = O.Q4Planar(*synth.q4_weight(97, 640, 61))
    x = synth.bf16_normal((3, 640), 62)
    a = O.q4_matmul(w, x, threads=3)
    b = O.f32_matmul(O.dequant_planar(w), O.bf16_to_f32(x), threads=2)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
