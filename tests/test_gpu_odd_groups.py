"""Few-token (5 <= m < 64) calls whose K is an odd number of 64-groups (K % 128 == 64) against the oracle.

The few-token kernel works in 128-column pieces.  With an odd group count, the last piece of the last K
slab holds one group: its other half re-reads the live half's words, meets zero X and a zero scale and bias,
and the scale/bias pairs come in 2-byte loads (a row's pairs are not 4-byte aligned).  Shapes: one group
(K = 64), 3 and 31 groups in one slab, 33 groups (a second slab of one half piece), and 43 groups (the
down projection of one GPU's share of config 1 under 4-way tensor parallelism, K = 2752); plain outputs,
bias and bf16 accumulate epilogues, the fused QKV, the MLP with its in-launch split-K reduction (bit-compared
with the separate reduction launch) and the norm-fused calls.  The reference's kernels take any K that is a
multiple of 64 (q4_gemm_and_moe.metal:2173-2486).
"""
import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("m", [5, 16, 24, 63])
@pytest.mark.parametrize("n,k", [(300, 64), (77, 192), (130, 1984), (96, 2112), (200, 2752)])
def test_linear_odd_group_count(kq, m, n, k):
    s = synth()
    case(f"few-token linear m={m} n={n} k={k} ({k // 64} groups)")
    wq = s.q4_weight(n, k, 5000 + n + k)
    x = s.bf16_normal((m, k), 5100 + m)
    W = q4_dev(kq, wq)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    y = kq.q4_linear(W, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, want, what=f"f32 m={m} k={k}")
    r0 = s.bf16_normal((m, n), 5200 + m)
    r = dev_bf16(r0).clone()
    kq.q4_linear(W, dev_bf16(x), y=r, accumulate=True)
    assert_bf16_rounded_close(host_bits(r), O.bf16_to_f32(r0) + want, rms(want), what=f"bf16 acc m={m} k={k}")


@pytest.mark.parametrize("m", [6, 16, 40])
@pytest.mark.parametrize("k", [192, 1984])
def test_qkv_bias_odd_group_count(kq, m, k):
    s = synth()
    case(f"few-token qkv with bias m={m} k={k}")
    shapes = ((k, k), (64, k), (64, k))
    wq = [s.q4_weight(n, kk, 5300 + i) for i, (n, kk) in enumerate(shapes)]
    bq = [s.bf16_normal((n,), 5310 + i, std=0.1) for i, (n, _) in enumerate(shapes)]
    x = s.bf16_normal((m, k), 5320 + m)
    got = kq.qkv(*(q4_dev(kq, w) for w in wq), dev_bf16(x), *(dev_bf16(b) for b in bq), out_dtype=kq.DTYPE_F32)
    for name, g_, w_, b_ in zip("qkv", got, wq, bq):
        want = O.q4_matmul(O.Q4Planar(*w_), x) + O.bf16_to_f32(b_)
        assert_rms_close(g_.cpu().numpy(), want, what=f"{name} m={m} k={k}")


@pytest.mark.parametrize("m", [5, 16, 24])
@pytest.mark.parametrize("hidden,inter", [(1984, 2752), (2048, 2752), (192, 4160)])
def test_mlp_odd_group_count(kq, m, hidden, inter):
    """The gate/up over an odd hidden and the down projection over an odd intermediate (split-K slabs
    whose last piece is half), in-launch reduction and the separate reduction launch bit for bit."""
    s = synth()
    case(f"few-token mlp m={m} hidden={hidden} inter={inter}")
    g, u = s.q4_weight(inter, hidden, 5400), s.q4_weight(inter, hidden, 5401)
    d = s.q4_weight(hidden, inter, 5402)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    h0 = s.bf16_normal((m, hidden), 5410 + m)
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    x = dev_bf16(h0)
    outs = {}
    try:
        for tk in (1, 0):
            kq.set_option(kq.OPT_SPLITK_TICKETS, tk)
            h = torch.zeros((m, hidden), dtype=torch.float32, device="cuda")
            kq.mlp(G, U, D, h, x=x)
            outs[tk] = h.cpu().numpy()
    finally:
        kq.set_option(kq.OPT_SPLITK_TICKETS, 1)
    assert_rms_close(outs[1], delta, what=f"mlp m={m} hidden={hidden} inter={inter}")
    assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32))
    hb = dev_bf16(h0).clone()
    kq.mlp(G, U, D, hb)
    assert_bf16_rounded_close(host_bits(hb), O.bf16_to_f32(h0) + delta, rms(delta), rel=1e-2,
                              what=f"mlp bf16 residual m={m}")


def rmsnorm_np(h_bits, ln_bits, eps=1e-6):
    """bf16(x * rsqrt(mean(x^2) + eps) * w), kr_rmsnorm's result (transformer_glue.metal:158-205)."""
    xf, wf = O.bf16_to_f32(h_bits), O.bf16_to_f32(ln_bits)
    r = 1.0 / np.sqrt((xf.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + eps)
    return O.f32_to_bf16((xf * r * wf).astype(np.float32))


@pytest.mark.parametrize("m", [9, 16])
def test_fused_norm_odd_group_count(kq, m):
    """The few-token kernel's per-wave RMSNorm over a row of 31 groups (zero X past K in the last piece)."""
    s = synth()
    H, I = 1984, 2752
    case(f"fused rmsnorm + qkv / mlp at H={H}, m={m}")
    h0 = s.bf16_normal((m, H), 5500 + m, std=3.0)
    ln = O.f32_to_bf16(1.0 + O.bf16_to_f32(s.bf16_normal((H,), 5501, std=0.1)))
    x = rmsnorm_np(h0, ln)
    shapes = ((H, H), (128, H), (128, H))
    wq = [s.q4_weight(n, k, 5502 + i) for i, (n, k) in enumerate(shapes)]
    got = kq.rmsnorm_qkv(dev_bf16(h0), dev_bf16(ln), 1e-6, *(q4_dev(kq, w) for w in wq), out_dtype=kq.DTYPE_F32)
    for name, g_, w_ in zip("qkv", got, wq):
        assert_rms_close(g_.cpu().numpy(), O.q4_matmul(O.Q4Planar(*w_), x), what=f"fused {name} m={m}")
    gw, uw = s.q4_weight(I, H, 5510), s.q4_weight(I, H, 5511)
    dw = s.q4_weight(H, I, 5512)
    delta = O.q4_mlp(O.Q4Planar(*gw), O.Q4Planar(*uw), O.Q4Planar(*dw), x)
    hd = dev_bf16(h0).clone()
    kq.rmsnorm_mlp(q4_dev(kq, gw), q4_dev(kq, uw), q4_dev(kq, dw), hd, dev_bf16(ln), 1e-6)
    assert_bf16_rounded_close(host_bits(hd), O.bf16_to_f32(h0) + delta, rms(delta), rel=1e-2,
                              what=f"fused mlp m={m}")
