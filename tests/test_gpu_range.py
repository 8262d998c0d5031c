"""Activations outside fp16's range through the batched kernels.

The reference keeps fp32 tiles for 1 < M < 64 (kernels/metal/
q4_gemm_and_moe.metal:2186-2187) and stages half for M >= 64.  Here the
few-token kernel (2 <= m < 64, more than 16 rows in 16-row chunks) multiplies
bf16 x by bf16 (128 + q) with f32 accumulation, exact for every bf16 value, so
each token row meets the bar on its own.  The prefill kernel (m >= 64) stages x
in fp16 like the reference: a tile whose accumulators overflow (|x| > 65504)
is recomputed in f32, so huge rows stay exact; rows below fp16's normal range
(RMS under 2^-14) keep fp16's subnormal precision and are held to the bar of
the whole output only.

Inputs: bf16 activations with magnitudes log-uniform over 1e-6 .. 1e5 per
element, and rows of N(0, 1) scaled by 10^k, k = -6 .. 5 (tiny and huge rows
side by side).  Bars: max |gpu - oracle| <= 1e-2 * RMS(oracle) over the
output, and the same bar per token row against that row's RMS (a tiny row
cannot hide behind the huge ones)."""
import numpy as np
import pytest

import oracle as O
from _util import assert_rms_close, dev_bf16, q4_dev, rms

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)


def wide_activations(m, k, seed, kind):
    rng = np.random.default_rng(seed)
    if kind == "per_element":
        mag = 10.0 ** rng.uniform(-6, 5, size=(m, k))
        x = mag * rng.choice([-1.0, 1.0], size=(m, k))
    else:  # rows of N(0, 1) times 10^k, k cycling through -6 .. 5
        x = rng.standard_normal((m, k)) * (10.0 ** (np.arange(m) % 12 - 6))[:, None]
    return O.f32_to_bf16(x.astype(np.float32))


FP16_MIN_NORMAL = 2.0 ** -14


def check_rows(got, want, what, x=None):
    """Whole-output bar, then the bar per row; with `x` (an fp16-staged m >= 64 launch) rows whose
    RMS is below fp16's normal range are left to the whole-output bar."""
    assert_rms_close(got, want, what=what)
    for i in range(want.shape[0]):
        if x is not None and rms(O.bf16_to_f32(x[i])) < FP16_MIN_NORMAL:
            continue
        assert_rms_close(got[i], want[i], what=f"{what} row {i}")


def staged_fp16(m, x):
    return x if m >= 64 else None


@pytest.mark.parametrize("kind", ["per_element", "per_row"])
@pytest.mark.parametrize("m", [5, 16, 48, 512])
def test_linear_wide_activations(kq, m, kind):
    from kriya_q4 import synth
    n, k = 384, 2048
    case(f"linear with activations over 1e-6..1e5 ({kind}) m={m} n={n} k={k}")
    wq = synth.q4_weight(n, k, 7600 + m)
    x = wide_activations(m, k, 7601 + m, kind)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    got = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    check_rows(got, want, f"linear m={m} {kind}", staged_fp16(m, x))


@pytest.mark.parametrize("m", [9, 16, 40, 256])
def test_gate_up_and_split_k_wide_activations(kq, m):
    """gate/up with the SwiGLU epilogue, and a K = 11008 projection (split over K slabs; at m <= 16
    without a workspace it runs on the tiled kernel, which stages each row times a power of two)."""
    from kriya_q4 import synth
    case(f"gate/up and K-split linear with per-row scaled activations m={m}")
    H, I = 1024, 1536
    g, u = synth.q4_weight(I, H, 7701), synth.q4_weight(I, H, 7702)
    x = wide_activations(m, H, 7703 + m, "per_row")
    want = O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x)
    got = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    check_rows(got, want, f"gate/up m={m}", staged_fp16(m, x))
    d = synth.q4_weight(512, 11008, 7704)
    xd = wide_activations(m, 11008, 7705 + m, "per_row")
    want = O.q4_matmul(O.Q4Planar(*d), xd)
    got = kq.q4_linear(q4_dev(kq, d), dev_bf16(xd), out_dtype=kq.DTYPE_F32).cpu().numpy()
    check_rows(got, want, f"K-split linear m={m}", staged_fp16(m, xd))


def test_moe_grouped_wide_activations(kq):
    """Grouped experts (T * K > 16) on the few-token kernel."""
    from kriya_q4 import synth
    T, E, K, H, I = 24, 8, 2, 512, 384
    case(f"moe grouped experts with per-row scaled activations T={T}")
    g, u = synth.q4_weight(E * I, H, 7801), synth.q4_weight(E * I, H, 7802)
    d = synth.q4_weight(E * H, I, 7803)
    x = wide_activations(T, H, 7804, "per_row")
    logits = synth.f32_normal((T, E), 7805)
    route = O.moe_route(logits, K, True)
    want = O.moe_experts(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), E, x, route[0], route[1])
    import torch
    r = kq.moe_route(torch.from_numpy(logits).cuda(), K, True)
    got = kq.moe_experts(q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d), E, dev_bf16(x), r).cpu().numpy()
    check_rows(got, want, "moe grouped")
