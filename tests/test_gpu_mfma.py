"""GPU parity of the batched (m > 1) matrix-core path against the CPU oracle:
prefill GEMM (config 2: the seven projections of one Qwen2.5-3B layer at
M = 512), fused gate/up SwiGLU epilogue, fused QKV with bias, batched-decode
shapes (config 1 B = 4, 16) and the split-K reduction.

Bar: max |gpu - oracle| <= 1e-2 * RMS(oracle) on f32 outputs; bf16 outputs are
the RNE of an f32 value within 1e-3 * RMS of the oracle.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "closed_form.npz"))


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


def test_gemm_reference_fixture_64x64x128(kq):
    case("mfma gemm fixture M=64 N=64 K=128 (test_shader_compile.rs:1598)")
    w = q4_dev(kq, (FIX["gemm_64x64x128_qw"], FIX["gemm_64x64x128_sc"], FIX["gemm_64x64x128_bi"]))
    x = dev_bf16(FIX["gemm_64x64x128_x"])
    want = FIX["gemm_64x64x128_y"]
    y = kq.q4_linear(w, x, out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert np.max(np.abs(y - want)) < 0.05
    assert_rms_close(y, want, what="gemm fixture")
    yb = kq.q4_linear(w, x, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb), want, rms(want), what="gemm fixture bf16")


@pytest.mark.parametrize("m,n,k", [(2, 300, 128), (4, 2048, 2048), (16, 1000, 2048), (3, 200, 192), (7, 96, 512),
                                   (9, 40, 1408), (17, 64, 64), (33, 130, 192),
                                   (64, 256, 1408), (100, 384, 512), (129, 96, 2048 + 64)])
def test_linear_batched_shapes(kq, m, n, k):
    s = synth()
    case(f"mfma linear m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 3000 + m + n)
    x = s.bf16_normal((m, k), 3100 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    y = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, want, what=f"m={m} n={n} k={k}")
    # accumulate into a bf16 residual
    r0 = s.bf16_normal((m, n), 3200 + m)
    r = dev_bf16(r0).clone()
    kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), y=r, accumulate=True)
    assert_bf16_rounded_close(host_bits(r), O.bf16_to_f32(r0) + want, rms(want), what=f"acc m={m}")


@pytest.mark.parametrize("m,n", [(3, 77), (5, 77), (9, 33), (17, 45)])
def test_linear_accumulate_bf16_odd_element_count(kq, m, n):
    """bf16 accumulate where m * n is odd: the last element has no partner in a 32-bit pair, so the
    epilogue must read exactly the element it updates (the output tensor ends right after it)."""
    s = synth()
    k = 256
    case(f"bf16 accumulate, odd element count m={m} n={n}")
    wq = s.q4_weight(n, k, 3300 + m + n)
    x = s.bf16_normal((m, k), 3310 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    r0 = s.bf16_normal((m, n), 3320 + m)
    r = dev_bf16(r0).clone()
    kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), y=r, accumulate=True)
    assert_bf16_rounded_close(host_bits(r), O.bf16_to_f32(r0) + want, rms(want), what=f"acc m={m} n={n}")


CFG2 = [("q", 2048, 2048, 2001), ("k", 256, 2048, 2002), ("v", 256, 2048, 2003), ("o", 2048, 2048, 2004),
        ("gate", 11008, 2048, 2005), ("up", 11008, 2048, 2006), ("down", 2048, 11008, 2007)]


@pytest.mark.parametrize("name,n,k,seed", CFG2)
def test_prefill_config2_projection(kq, name, n, k, seed):
    s = synth()
    case(f"cfg2 prefill {name} [{n},{k}] M=512")
    wq = s.q4_weight(n, k, seed)
    x = s.bf16_normal((512, k), seed + 100)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    y = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    err = assert_rms_close(y, want, what=f"cfg2 {name}")
    print(f"cfg2 {name}: max err {err / rms(want):.2e} of rms", flush=True)


@pytest.mark.parametrize("m", [4, 16, 64, 512])
def test_gate_up_batched(kq, m):
    s = synth()
    case(f"mfma gate_up swiglu m={m} [11008,2048]")
    g, u = s.q4_weight(11008, 2048, 2005), s.q4_weight(11008, 2048, 2006)
    x = s.bf16_normal((m, 2048), 2300 + m)
    want = O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x)
    a = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(a, want, what=f"gate_up m={m}")


@pytest.mark.parametrize("m", [1, 3, 16, 512])
def test_qkv_with_bias(kq, m):
    s = synth()
    case(f"qkv with bias m={m}")
    ws = [s.q4_weight(n, 2048, 2400 + i) for i, n in enumerate((2048, 256, 256))]
    bs = [s.bf16_normal((n,), 2410 + i, std=0.1) for i, n in enumerate((2048, 256, 256))]
    x = s.bf16_normal((m, 2048), 2420 + m)
    outs = kq.qkv(*(q4_dev(kq, w) for w in ws), dev_bf16(x), *(dev_bf16(b) for b in bs), out_dtype=kq.DTYPE_F32)
    for i, name in enumerate("qkv"):
        want = O.q4_matmul(O.Q4Planar(*ws[i]), x) + O.bf16_to_f32(bs[i])[None, :]
        assert_rms_close(outs[i].cpu().numpy(), want, what=f"{name} m={m}")
    outs_b = kq.qkv(*(q4_dev(kq, w) for w in ws), dev_bf16(x), *(dev_bf16(b) for b in bs), out_dtype=kq.DTYPE_BF16)
    want = O.q4_matmul(O.Q4Planar(*ws[1]), x) + O.bf16_to_f32(bs[1])[None, :]
    assert_bf16_rounded_close(host_bits(outs_b[1]), want, rms(want), what=f"k bf16 m={m}")


def test_mlp_batched_split_k_is_deterministic(kq):
    s = synth()
    case("mlp B=16 (split-K down projection): two runs bitwise equal, vs oracle")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    d = s.q4_weight(2048, 11008, 1003)
    h0 = s.bf16_normal((16, 2048), 1026)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    runs = []
    for _ in range(2):
        h = torch.from_numpy(O.bf16_to_f32(h0)).cuda()
        kq.mlp(G, U, D, h, x=dev_bf16(h0))
        runs.append(h.cpu().numpy())
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))
    assert_rms_close(runs[0] - O.bf16_to_f32(h0), delta, what="mlp B=16")


@pytest.mark.parametrize("m,n,k", [(17, 200, 256), (40, 72, 640), (130, 300, 128), (33, 48, 192), (70, 130, 320)])
def test_gate_up_prefill_tails(kq, m, n, k):
    """m > 16 runs the prefill kernel: token-row and weight-row tails that end inside a tile; k = 192
    and 320 (odd group counts) take the 64-column steps, the others 128-column steps."""
    s = synth()
    case(f"prefill gate_up tails m={m} n={n} k={k}")
    g, u = s.q4_weight(n, k, 2500 + n), s.q4_weight(n, k, 2501 + n)
    x = s.bf16_normal((m, k), 2502 + m)
    want = O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x)
    a = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(a, want, what=f"gate_up m={m} n={n}")
    ab = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(ab), want, rms(want), what=f"gate_up bf16 m={m}")


def test_mlp_prefill_split_k(kq):
    """m = 96: the down projection's few tiles are split over K (f32 partials summed in split order)."""
    s = synth()
    case("mlp m=96 hidden 512 inter 1408: prefill kernels with split-K down, deterministic, vs oracle")
    g, u = s.q4_weight(1408, 512, 2601), s.q4_weight(1408, 512, 2602)
    d = s.q4_weight(512, 1408, 2603)
    h0 = s.bf16_normal((96, 512), 2604)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    runs = []
    for _ in range(2):
        h = torch.from_numpy(O.bf16_to_f32(h0)).cuda()
        kq.mlp(G, U, D, h, x=dev_bf16(h0))
        runs.append(h.cpu().numpy())
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))
    assert_rms_close(runs[0] - O.bf16_to_f32(h0), delta, what="mlp m=96")


def test_splitk_reduction_paths_bitwise(kq):
    """The split-K reduction has a vector form (eight outputs per thread, 16-byte aligned rows) and a
    scalar form (an output that is not 16-byte aligned); both add the partials in split order from 0,
    so an h offset by one f32 element gives the same bits as an aligned one."""
    s = synth()
    case("mlp m=96 split-K down: h 16-byte aligned vs offset by one element, bitwise")
    g, u = s.q4_weight(1408, 512, 2611), s.q4_weight(1408, 512, 2612)
    d = s.q4_weight(512, 1408, 2613)
    h0 = s.bf16_normal((96, 512), 2614)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    outs = []
    for off in (0, 1):
        buf = torch.zeros(96 * 512 + 4, dtype=torch.float32, device="cuda")
        h = buf[off:off + 96 * 512].view(96, 512)
        h.copy_(torch.from_numpy(O.bf16_to_f32(h0)).cuda())
        assert (h.data_ptr() % 16 == 0) == (off == 0)
        kq.mlp(G, U, D, h, x=dev_bf16(h0))
        outs.append(h.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("m", [64, 512])
def test_prefill_kernels_agree(kq, m):
    """The register-dequant prefill kernel and the LDS-dequant tiled kernel give the same sums
    up to f32 summation order."""
    s = synth()
    case(f"prefill vs tiled kernel m={m} [2048, 2048]")
    wq = s.q4_weight(2048, 2048, 2700)
    x = dev_bf16(s.bf16_normal((m, 2048), 2701))
    w = q4_dev(kq, wq)
    lib = kq.lib()
    outs = {}
    try:
        for opt in (1, 2):  # the tiled kernel; the prefill kernel with 64-column steps
            assert lib.kr_set_option(kq.OPT_PREFILL_KERNEL, opt) == 0
            outs[opt] = kq.q4_linear(w, x, out_dtype=kq.DTYPE_F32).cpu().numpy()
    finally:
        lib.kr_set_option(kq.OPT_PREFILL_KERNEL, 0)
    got = kq.q4_linear(w, x, out_dtype=kq.DTYPE_F32).cpu().numpy()
    for opt, ref in outs.items():
        assert np.max(np.abs(got - ref)) <= 1e-4 * rms(ref), f"option {opt}"


@pytest.mark.parametrize("m", [64, 200])
def test_mlp_prefill_operands_bitwise(kq, m):
    """kr_q4_mlp at m >= 64 converts x to the prefill kernel's fp16 operands once and has the gate/up
    launch write the activation in that form for the down projection: the same bits as every block
    converting its own X slices (option 0), also when x overflows fp16 (the blocks whose sums do not
    stay finite recompute their tiles in f32 from the bf16 operands) -- against the oracle as well."""
    s = synth()
    case(f"mlp m={m} hidden 512 inter 1408: pre-converted fp16 operands vs per-block conversion")
    g, u = s.q4_weight(1408, 512, 2801), s.q4_weight(1408, 512, 2802)
    d = s.q4_weight(512, 1408, 2803)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    lib = kq.lib()
    xs = {"normal": s.bf16_normal((m, 512), 2804 + m)}
    big = O.bf16_to_f32(xs["normal"]).copy()
    big[3] *= 1e5  # a row beyond fp16's range (65504)
    xs["overflow"] = O.f32_to_bf16(big)
    for name, x in xs.items():
        res = {}
        try:
            for opt in (0, 1):
                assert lib.kr_set_option(kq.OPT_PREFILL_OPERANDS, opt) == 0
                h = torch.zeros((m, 512), dtype=torch.float32, device="cuda")
                kq.mlp(G, U, D, h, x=dev_bf16(x))
                res[opt] = h.cpu().numpy()
        finally:
            lib.kr_set_option(kq.OPT_PREFILL_OPERANDS, 1)
        assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32)), name
        want = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), x)
        assert np.all(np.isfinite(res[1])), name
        for i in range(m):
            assert_rms_close(res[1][i], want[i], what=f"mlp {name} row {i}")


@pytest.mark.parametrize("m", [17, 24, 32, 33, 48, 63])
def test_skinny_row_groups_bitwise(kq, m):
    """The few-token kernel at 17 <= m <= 63 runs 32-row launches that multiply every unpacked weight
    word with two 16-row groups of x (option 2, the default): the same bits as 16-row launches
    (option 1) for the plain, accumulating, gate/up, QKV (with bias, and with the RMSNorm staged in
    the kernel) and MLP (split K with the in-launch reduction) calls, and within the bar of the
    oracle."""
    s = synth()
    lib = kq.lib()
    case(f"few-token row groups m={m}: 32-row launches vs 16-row launches")
    w = s.q4_weight(1000, 2048, 3101)
    gw, uw = s.q4_weight(700, 1536, 3102), s.q4_weight(700, 1536, 3103)
    qw, kw, vw = s.q4_weight(512, 1024, 3104), s.q4_weight(128, 1024, 3105), s.q4_weight(128, 1024, 3106)
    mg, mu, md = s.q4_weight(4608, 512, 3107), s.q4_weight(4608, 512, 3108), s.q4_weight(512, 4608, 3109)
    W, GW, UW, QW, KW, VW, MG, MU, MD = (q4_dev(kq, t) for t in (w, gw, uw, qw, kw, vw, mg, mu, md))
    x = s.bf16_normal((m, 2048), 3110 + m)
    xg = s.bf16_normal((m, 1536), 3111 + m)
    xq = s.bf16_normal((m, 1024), 3112 + m)
    xm = s.bf16_normal((m, 512), 3113 + m)
    qb, kb, vb = (dev_bf16(s.bf16_normal((n,), 3114 + n)) for n in (512, 128, 128))
    ln = dev_bf16(s.bf16_normal((1024,), 3115))
    y0 = s.bf16_normal((m, 1000), 3116 + m)
    res = {}
    try:
        for opt in (1, 2):
            assert lib.kr_set_option(kq.OPT_SKINNY_GROUPS, opt) == 0
            r = {}
            r["linear"] = kq.q4_linear(W, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
            ya = dev_bf16(y0)
            kq.q4_linear(W, dev_bf16(x), y=ya, accumulate=True)
            r["accumulate"] = host_bits(ya)
            r["gate_up"] = kq.gate_up_act(GW, UW, dev_bf16(xg), out_dtype=kq.DTYPE_F32).cpu().numpy()
            r["qkv"] = [t.cpu().numpy() for t in kq.qkv(QW, KW, VW, dev_bf16(xq), qb, kb, vb)]
            r["rmsnorm_qkv"] = [t.cpu().numpy() for t in kq.rmsnorm_qkv(dev_bf16(xq), ln, 1e-6, QW, KW, VW, qb, kb, vb)]
            h = torch.zeros((m, 512), dtype=torch.float32, device="cuda")
            kq.mlp(MG, MU, MD, h, x=dev_bf16(xm))
            r["mlp"] = h.cpu().numpy()
            res[opt] = r
    finally:
        lib.kr_set_option(kq.OPT_SKINNY_GROUPS, 2)
    for name in res[1]:
        a, b = res[1][name], res[2][name]
        for u, v in zip(a if isinstance(a, list) else [a], b if isinstance(b, list) else [b]):
            assert np.array_equal(np.ascontiguousarray(u).view(np.uint8), np.ascontiguousarray(v).view(np.uint8)), name
    assert_rms_close(res[2]["linear"], O.q4_matmul(O.Q4Planar(*w), x), what=f"linear m={m}")
    want_acc = O.bf16_to_f32(y0).astype(np.float64) + O.q4_matmul(O.Q4Planar(*w), x)
    got_acc = O.bf16_to_f32(res[2]["accumulate"]).astype(np.float64)
    assert np.all(np.abs(got_acc - want_acc) <= np.abs(want_acc) * 2.0 ** -8 + 1e-2 * rms(want_acc))
    want_mlp = O.q4_mlp(O.Q4Planar(*mg), O.Q4Planar(*mu), O.Q4Planar(*md), xm)
    assert_rms_close(res[2]["mlp"], want_mlp, what=f"mlp m={m}")


@pytest.mark.parametrize("m", [5, 16, 24])
def test_skinny_depth_bitwise(kq, m):
    """The few-token kernel's register ring (two tiles in flight, chosen for runs of >= 6 tiles, or
    forced with KR_OPT_SKINNY_DEPTH) gives the same bits as one tile in flight: gate/up and plain
    launches whose runs hold 1..6 tiles with ragged ends, one and two row groups, and the MLP (its
    split-K down projection reduces inside the launch); the default against the oracle too."""
    s = synth()
    lib = kq.lib()
    case(f"few-token ring depth m={m}: depth 2 vs 3 vs automatic")
    shapes = [(11008, 2048), (10995, 2048), (300, 1024), (3000, 1536)]
    mats = [(s.q4_weight(n, k, 3201 + i), s.q4_weight(n, k, 3301 + i)) for i, (n, k) in enumerate(shapes)]
    dev = [(q4_dev(kq, g), q4_dev(kq, u)) for g, u in mats]
    xs = [s.bf16_normal((m, k), 3401 + i + m) for i, (_, k) in enumerate(shapes)]
    mg, mu, md = s.q4_weight(4608, 512, 3501), s.q4_weight(4608, 512, 3502), s.q4_weight(512, 4608, 3503)
    MG, MU, MD = (q4_dev(kq, t) for t in (mg, mu, md))
    xm = s.bf16_normal((m, 512), 3504 + m)
    res = {}
    try:
        for opt in (2, 3, 0):
            assert lib.kr_set_option(kq.OPT_SKINNY_DEPTH, opt) == 0
            r = []
            for (G, U), x in zip(dev, xs):
                r.append(kq.gate_up_act(G, U, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy())
                r.append(host_bits(kq.gate_up_act(G, U, dev_bf16(x), out_dtype=kq.DTYPE_BF16)))
                r.append(kq.q4_linear(G, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy())
            h = torch.zeros((m, 512), dtype=torch.float32, device="cuda")
            kq.mlp(MG, MU, MD, h, x=dev_bf16(xm))
            r.append(h.cpu().numpy())
            res[opt] = r
    finally:
        lib.kr_set_option(kq.OPT_SKINNY_DEPTH, 0)
    for opt in (3, 0):
        for i, (a, b) in enumerate(zip(res[2], res[opt])):
            assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8)), (opt, i)
    for i, ((g, u), x) in enumerate(zip(mats, xs)):
        assert_rms_close(res[0][3 * i], O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x), what=f"gate/up {shapes[i]}")
        assert_rms_close(res[0][3 * i + 2], O.q4_matmul(O.Q4Planar(*g), x), what=f"linear {shapes[i]}")
    assert_rms_close(res[0][-1], O.q4_mlp(O.Q4Planar(*mg), O.Q4Planar(*mu), O.Q4Planar(*md), xm), what="mlp")


def test_mlp_config2_full_shape(kq):
    """kr_q4_mlp at config 2's MLP shape (M = 512, hidden 2048, inter 11008; encoder.rs:2851-2906), the call
    bench.py times: the fused gate/up SwiGLU prefill epilogue, then the down projection split over K = 11008
    into f32 partials summed in split order.  Into an f32 residual, each row within 1e-2 of its own RMS against
    the oracle, and bit-identical with the fp16 operands converted once per call (option 1, the default) or
    per block (option 0)."""
    s = synth()
    M, H, I = 512, 2048, 11008
    case(f"mlp cfg2 full shape M={M} hidden {H} inter {I}, split-K down, both operand options")
    g, u, d = s.q4_weight(I, H, 2005), s.q4_weight(I, H, 2006), s.q4_weight(H, I, 2007)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    x = s.bf16_normal((M, H), 2105)
    h0 = O.bf16_to_f32(s.bf16_normal((M, H), 2106))
    ws = kq.mlp_workspace(M, H, I)
    lib = kq.lib()
    res = {}
    try:
        for opt in (0, 1):
            assert lib.kr_set_option(kq.OPT_PREFILL_OPERANDS, opt) == 0
            h = torch.from_numpy(h0).cuda()
            kq.mlp(G, U, D, h, x=dev_bf16(x), workspace=ws)
            res[opt] = h.cpu().numpy()
    finally:
        lib.kr_set_option(kq.OPT_PREFILL_OPERANDS, 1)
    assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), x)
    got = res[1].astype(np.float64) - h0
    worst = 0.0
    for i in range(M):
        worst = max(worst, assert_rms_close(got[i], delta[i], what=f"mlp cfg2 row {i}") / rms(delta[i]))
    print(f"mlp cfg2: worst row max err {worst:.2e} of the row's rms", flush=True)


def test_consolidated_qkv_matches_separate_projections(kq):
    """Restates test_shader_compile.rs:3185-3286: the q, k and v rows of one layer live in ONE Q4_G64 buffer
    (192 x 64, weights ((idx % 31) - 15) * 0.02 quantised by quantize_f32_to_q4_group64), bound to the device
    from its split planes with the nibble plane used in place; the fused QKV call over its three row ranges
    passes the reference's own check (|f32 dot of the dequantised q rows with the f32 input - the bf16
    output| < 0.05) and gives the bits of the three separate projections."""
    k, q_dim, kv_dim = 64, 64, 64
    total = q_dim + 2 * kv_dim
    case("consolidated qkv 192 x 64 from split planes in place vs separate projections")
    wflat = ((np.arange(total * k) % 31).astype(np.float32) - np.float32(15.0)) * np.float32(0.02)
    blocks = O.quantize_q4_g64(wflat)
    qs, sb = O.split_blocks36(blocks)
    qs_dev = torch.from_numpy(qs.ravel().copy()).cuda()
    sb_dev = torch.from_numpy(sb.view(np.uint8).ravel().copy()).cuda()
    W = kq.Q4Matrix.from_split(qs_dev, sb_dev, total, k, in_place=True)
    assert W.qw.data_ptr() == qs_dev.data_ptr()
    inp = np.sin(np.arange(k, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    x = O.f32_to_bf16(inp)[None, :]
    ranges = ((0, q_dim), (q_dim, q_dim + kv_dim), (q_dim + kv_dim, total))
    outs = kq.qkv(*(W.rows(lo, hi) for lo, hi in ranges), dev_bf16(x), out_dtype=kq.DTYPE_BF16)
    deq = O.dequant_blocks36(blocks).reshape(total, k)
    out_q = O.bf16_to_f32(host_bits(outs[0]).ravel())
    for row in range(q_dim):
        dot = np.float32(0.0)
        for c in range(k):  # the reference's sequential f32 dot
            dot = np.float32(dot + deq[row, c] * inp[c])
        assert abs(float(dot) - float(out_q[row])) < 0.05, f"q row {row}: cpu {dot} gpu {out_q[row]}"
    for i, (lo, hi) in enumerate(ranges):
        sep = kq.q4_linear(W.rows(lo, hi), dev_bf16(x), out_dtype=kq.DTYPE_BF16)
        assert np.array_equal(host_bits(sep), host_bits(outs[i])), f"projection {i}"


@pytest.mark.parametrize("m", [1, 16, 512])
def test_consolidated_qkv_config3_shape(kq, m):
    """Config 3's attention projections (q [2048, 2048], k and v [256, 2048], with bf16 biases) concatenated in
    one buffer that is bound from split planes in place: the row-range views give the bits of separately bound
    matrices, and the oracle's results within the bar."""
    s = synth()
    case(f"consolidated qkv cfg3 shape from split planes, m={m}")
    shapes = (2048, 256, 256)
    parts = [s.q4_weight(n, 2048, 2440 + i) for i, n in enumerate(shapes)]
    cat = O.Q4Planar(*(np.concatenate([p[j] for p in parts]) for j in range(3)))
    qs, sb = O.split_blocks36(O.planar_to_blocks36(cat))
    qs_dev = torch.from_numpy(qs.ravel().copy()).cuda()
    sb_dev = torch.from_numpy(sb.view(np.uint8).ravel().copy()).cuda()
    W = kq.Q4Matrix.from_split(qs_dev, sb_dev, cat.n, 2048, in_place=True)
    bs = [s.bf16_normal((n,), 2450 + i, std=0.1) for i, n in enumerate(shapes)]
    x = s.bf16_normal((m, 2048), 2460 + m)
    bounds = np.cumsum((0,) + shapes)
    views = [W.rows(int(bounds[i]), int(bounds[i + 1])) for i in range(3)]
    got = kq.qkv(*views, dev_bf16(x), *(dev_bf16(b) for b in bs), out_dtype=kq.DTYPE_F32)
    sep = kq.qkv(*(q4_dev(kq, p) for p in parts), dev_bf16(x), *(dev_bf16(b) for b in bs), out_dtype=kq.DTYPE_F32)
    for i, name in enumerate("qkv"):
        assert torch.equal(got[i].view(torch.int32), sep[i].view(torch.int32)), name
        want = O.q4_matmul(O.Q4Planar(*parts[i]), x) + O.bf16_to_f32(bs[i])[None, :]
        assert_rms_close(got[i].cpu().numpy(), want, what=f"{name} m={m}")


@pytest.mark.parametrize("opt", [0, 2])
def test_prefill_fp16_overflow_fallback_k2048(kq, opt):
    """x beyond fp16's range (65504) sends a prefill block to its exact f32 fallback, chosen by a block-wide
    OR whose flag bytes sit in an X buffer.  With 64-column steps (option 2) K = 2048 has 32 steps, so the
    last step's clamped look-ahead slice goes to buffer (32 + 1) % 3 = 0, where the flags are: the
    fallback still triggers for the overflowing rows' blocks, and no block takes it by mistake (every row
    within the bar of the oracle, also without overflow)."""
    s = synth()
    m, n, k = 64, 256, 2048
    case(f"prefill fp16-overflow fallback, option {opt}, m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 2720)
    x = s.bf16_normal((m, k), 2721)
    big = O.bf16_to_f32(x).copy()
    big[5] *= 1e5
    xs = {"normal": x, "overflow": O.f32_to_bf16(big)}
    w = q4_dev(kq, wq)
    lib = kq.lib()
    try:
        assert lib.kr_set_option(kq.OPT_PREFILL_KERNEL, opt) == 0
        for name, xv in xs.items():
            want = O.q4_matmul(O.Q4Planar(*wq), xv)
            got = kq.q4_linear(w, dev_bf16(xv), out_dtype=kq.DTYPE_F32).cpu().numpy()
            assert np.all(np.isfinite(got)), name
            for i in range(m):
                assert_rms_close(got[i], want[i], what=f"{name} row {i}")
    finally:
        lib.kr_set_option(kq.OPT_PREFILL_KERNEL, 0)


@pytest.mark.parametrize("m,hidden,inter", [(512, 2048, 11008), (96, 512, 1408), (200, 1024, 2816)])
def test_prefill_xcd_split_bitwise(kq, m, hidden, inter):
    """kr_q4_mlp's split-K down projection places each K split on its own XCDs (KR_OPT_PREFILL_XCD_SPLIT = 1,
    the default): a different block order over the same (tile, split) pairs, so the same bits as the default
    tile grouping (option 0), and within the bar of the oracle."""
    s = synth()
    case(f"prefill split K on per-split XCDs, mlp m={m} hidden={hidden} inter={inter}")
    g, u, d = s.q4_weight(inter, hidden, 2901), s.q4_weight(inter, hidden, 2902), s.q4_weight(hidden, inter, 2903)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    x = s.bf16_normal((m, hidden), 2904)
    ws = kq.mlp_workspace(m, hidden, inter)
    res = {}
    try:
        for opt in (0, 1):
            kq.set_option(kq.OPT_PREFILL_XCD_SPLIT, opt)
            h = torch.zeros((m, hidden), dtype=torch.float32, device="cuda")
            kq.mlp(G, U, D, h, x=dev_bf16(x), workspace=ws)
            res[opt] = h.cpu().numpy()
    finally:
        kq.set_option(kq.OPT_PREFILL_XCD_SPLIT, 1)
    assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))
    if m <= 200:
        want = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), x)
        for i in range(m):
            assert_rms_close(res[1][i], want[i], what=f"row {i}")
