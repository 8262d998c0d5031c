"""Seeded sweep of awkward shapes through every matmul entry point, against the oracle.

The entry points route by m, n and k to the decode GEMV (m = 1), the token GEMV (m = 2-4), the few-token
kernel (even or odd 64-group counts, one K slab or split K), the tiled and prefill kernels (m >= 17 / 64),
with or without a workspace.  A fixed pseudo-random draw of shapes (n from 1, k any multiple of 64 up to
5 slabs, m across every routing boundary) checks that each route gives the oracle's result within the
RMS bar: f32 outputs, bf16 accumulation, the fused QKV with biases, gate/up with its activation, and the MLP.
"""
import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu

M_VALUES = [1, 2, 3, 4, 5, 7, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 100]


def shapes(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        m = int(M_VALUES[i % len(M_VALUES)])
        n = int(rng.choice([1, 3, 16, 17, 64, 100, 129, 257, 600]))
        k = 64 * int(rng.integers(1, 5 * 32 + 1))  # up to 5 K slabs of 2048
        out.append((m, n, k))
    return out


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("m,n,k", shapes(71, 34))
def test_linear_sweep(kq, m, n, k):
    s = synth()
    case(f"linear sweep m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 7000 + m * 7 + n + k)
    x = s.bf16_normal((m, k), 7100 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    W, xd = q4_dev(kq, wq), dev_bf16(x)
    y = kq.q4_linear(W, xd, out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, want, what=f"linear m={m} n={n} k={k}")
    ws = kq.linear_workspace(m, n, k)
    r0 = s.bf16_normal((m, n), 7200 + m)
    r = dev_bf16(r0).clone()
    kq.q4_linear(W, xd, y=r, accumulate=True, workspace=ws)
    assert_bf16_rounded_close(host_bits(r), O.bf16_to_f32(r0) + want, rms(want), what=f"linear_ws acc m={m}")


@pytest.mark.parametrize("m,n,k", [(m, n, min(k, 4096)) for m, n, k in shapes(72, 17)])
def test_gate_up_and_mlp_sweep(kq, m, n, k):
    """gate/up [n, k] with SiLU, then the MLP with down [k, n] (hidden k, intermediate n)."""
    s = synth()
    n = 64 * ((n + 63) // 64)  # the intermediate is the down projection's K: whole groups
    case(f"gate/up + mlp sweep m={m} inter={n} hidden={k}")
    g, u, d = s.q4_weight(n, k, 7300), s.q4_weight(n, k, 7301), s.q4_weight(k, n, 7302)
    x = s.bf16_normal((m, k), 7310 + m)
    a = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(a, O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x, variant=0), what=f"gate/up m={m}")
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), x)
    h = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    kq.mlp(q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d), h, x=dev_bf16(x))
    assert_rms_close(h.cpu().numpy(), delta, what=f"mlp m={m} inter={n} hidden={k}")


@pytest.mark.parametrize("m,n,k", [(m, n, min(k, 4096)) for m, n, k in shapes(73, 17)])
def test_qkv_bias_sweep(kq, m, n, k):
    s = synth()
    case(f"qkv sweep m={m} q rows={n} k={k}")
    rows = (n, max(1, n // 4), max(1, n // 4))
    wq = [s.q4_weight(r, k, 7400 + i) for i, r in enumerate(rows)]
    bq = [s.bf16_normal((r,), 7410 + i, std=0.1) for i, r in enumerate(rows)]
    x = s.bf16_normal((m, k), 7420 + m)
    got = kq.qkv(*(q4_dev(kq, w) for w in wq), dev_bf16(x), *(dev_bf16(b) for b in bq), out_dtype=kq.DTYPE_F32)
    for name, g_, w_, b_ in zip("qkv", got, wq, bq):
        want = O.q4_matmul(O.Q4Planar(*w_), x) + O.bf16_to_f32(b_)
        assert_rms_close(g_.cpu().numpy(), want, what=f"{name} m={m} k={k}")
