"""GPU parity of the format kernels and the single-token (m == 1) GEMV family
against the CPU oracle, through the C ABI.

Bars: bit-exact for dequantisation and layout conversion; for matmul outputs
max |gpu - oracle| <= 1e-2 * RMS(oracle) on f32 outputs, bf16 outputs within
one bf16 ulp of RNE(oracle).  The reference's own tests use |gpu - cpu| < 0.05
(test_shader_compile.rs:642-645); that bound is checked too on its fixtures.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "closed_form.npz"))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


# ---------------------------------------------------------------- format kernels

def test_dequant_bit_exact_config0(kq):
    s = synth()
    case("dequant cfg0 11008x2048 seed 0")
    wq = s.q4_weight(11008, 2048, 0)
    got = kq.dequant(q4_dev(kq, wq)).cpu().numpy()
    want = O.dequant_planar(O.Q4Planar(*wq))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_bit_exact_extreme_scales(kq):
    case("dequant extreme bf16 scale/bias bit patterns")
    rng = np.random.default_rng(5)
    n, k = 64, 512
    qw = rng.integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.integers(0, 1 << 16, size=(n, k // 64), dtype=np.uint64).astype(np.uint16)
    bi = rng.integers(0, 1 << 16, size=(n, k // 64), dtype=np.uint64).astype(np.uint16)
    sc[0, :4] = [0x7F80, 0xFF80, 0x0001, 0x8000]  # inf, -inf, subnormal, -0
    bi[0, :4] = [0xFF80, 0x7F80, 0x8000, 0x0001]
    got = kq.dequant(q4_dev(kq, (qw, sc, bi))).cpu().numpy()
    want = O.dequant_planar(O.Q4Planar(qw, sc, bi))
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(np.where(both_nan, 0, got.view(np.uint32)), np.where(both_nan, 0, want.view(np.uint32)))


def test_blocks36_round_trip_on_gpu(kq):
    case("blocks36 -> planar -> blocks36, 1000 LCG blocks + patterns")
    lcg = np.array(KATS["lcg_blocks_1000"], np.uint8)  # 8 rows x 125 groups
    dev = torch.from_numpy(lcg.ravel().copy()).cuda()
    w = kq.Q4Matrix.from_blocks36(dev, 8, 125 * 64)
    ref = O.blocks36_to_planar(lcg, 8, 125 * 64)
    assert np.array_equal(w.qw.cpu().numpy().view(np.uint32), ref.qw)
    assert np.array_equal(w.scales.cpu().numpy().view(np.uint16), ref.scales)
    assert np.array_equal(w.biases.cpu().numpy().view(np.uint16), ref.biases)
    back = w.to_blocks36().cpu().numpy().reshape(-1, 36)
    assert np.array_equal(back, lcg)


def test_split_planes_on_gpu(kq):
    """Split planes (tensor.rs:117-211) -> planar on the GPU: bit-equal to the 36-byte path and to the
    oracle's split (pinned by the reference's split/rejoin KATs), copied or in place; planar -> split
    gives the oracle's planes back."""
    case("split planes <-> planar, 1000 LCG blocks (8 x 125 groups)")
    lcg = np.array(KATS["lcg_blocks_1000"], np.uint8)
    n, k = 8, 125 * 64
    qs, sb = O.split_blocks36(lcg)
    ref = kq.Q4Matrix.from_blocks36(torch.from_numpy(lcg.ravel().copy()).cuda(), n, k)
    for in_place in (False, True):
        qs_dev = torch.from_numpy(qs.ravel().copy()).cuda()
        sb_dev = torch.from_numpy(sb.view(np.uint8).ravel().copy()).cuda()
        w = kq.Q4Matrix.from_split(qs_dev, sb_dev, n, k, in_place=in_place)
        assert (w.qw.data_ptr() == qs_dev.data_ptr()) == in_place
        for a, b in ((w.qw, ref.qw), (w.scales, ref.scales), (w.biases, ref.biases)):
            assert torch.equal(a, b), f"in_place={in_place}"
    qs2, sb2 = ref.to_split()
    assert np.array_equal(qs2.cpu().numpy(), qs.ravel())
    assert np.array_equal(sb2.cpu().numpy().view(np.uint16), sb.ravel())
    with pytest.raises(kq.KrError):
        kq.Q4Matrix.from_split(qs_dev, sb_dev, n, 100)  # k not a multiple of 64


def test_blocks36_config0_planar_equivalence(kq):
    case("cfg0 planar -> blocks36 (oracle) -> planar (gpu)")
    wq = synth().q4_weight(11008, 2048, 0)
    blocks = O.planar_to_blocks36(O.Q4Planar(*wq))
    w = kq.Q4Matrix.from_blocks36(torch.from_numpy(blocks.ravel()).cuda(), 11008, 2048)
    assert np.array_equal(w.qw.cpu().numpy().view(np.uint32), wq[0])
    assert np.array_equal(w.scales.cpu().numpy().view(np.uint16), wq[1])


def test_f16_to_bf16_all_patterns(kq):
    case("f16 -> bf16, all 65536 patterns")
    h = np.arange(1 << 16, dtype=np.uint16)
    got = host_bits(kq.f16_to_bf16(torch.from_numpy(h.view(np.int16)).cuda()))
    want = np.array([O.half_to_bf16(int(v), True) for v in h], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- GEMV m == 1

@pytest.mark.parametrize("name", ["gemv_5x64", "gemv_7x128", "gemv_19x128", "persist_256"])
def test_gemv_reference_fixtures(kq, name):
    case(f"gemv fixture {name}")
    w = q4_dev(kq, (FIX[f"{name}_qw"], FIX[f"{name}_sc"], FIX[f"{name}_bi"]))
    x = dev_bf16(FIX[f"{name}_x"])
    want = FIX[f"{name}_y"]
    y32 = kq.q4_linear(w, x, out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
    assert np.max(np.abs(y32 - want)) < 0.05  # the reference test's own bound
    assert_rms_close(y32, want, what=name)
    yb = kq.q4_linear(w, x, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb)[0], want, rms(want), what=name)


def test_gemv_config0_full_size(kq):
    s = synth()
    case("gemv cfg0 11008x2048 seed 0, f32 and bf16 outputs")
    wq = s.q4_weight(11008, 2048, 0)
    x = s.bf16_normal((1, 2048), 1)
    w = q4_dev(kq, wq)
    y = kq.q4_linear(w, dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
    want = O.q4_matmul(O.Q4Planar(*wq), x)[0]
    gold = O.q4_matmul_f64(O.Q4Planar(*wq), x)[0]
    err = assert_rms_close(y, want, what="cfg0")
    print(f"cfg0: max|gpu-oracle| = {err:.3e} ({err / rms(want):.2e} of rms), "
          f"max|gpu-f64| = {np.max(np.abs(y - gold)):.3e}, max|oracle-f64| = {np.max(np.abs(want - gold)):.3e}")
    yb = kq.q4_linear(w, dev_bf16(x), out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb)[0], want, rms(want), what="cfg0 bf16")


@pytest.mark.parametrize("n,k", [(1, 64), (3, 128), (19, 512), (37, 1024), (73, 512), (129, 1408),
                                 (64, 11008), (2048, 11008), (300, 2048 + 64)])
def test_gemv_shapes(kq, n, k):
    s = synth()
    case(f"gemv n={n} k={k}")
    wq = s.q4_weight(n, k, 100 + n + k)
    x = s.bf16_normal((1, k), 200 + n)
    want = O.q4_matmul(O.Q4Planar(*wq), x)[0]
    for rpw in (1, 2, 4, 8):
        kq.set_option(kq.OPT_GEMV_ROWS_PER_WAVE, rpw)
        try:
            y = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
        finally:
            kq.set_option(kq.OPT_GEMV_ROWS_PER_WAVE, 2)
        assert_rms_close(y, want, what=f"n={n} k={k} rows/wave={rpw}")


@pytest.mark.parametrize("n,k", [(37, 4160), (2048, 11008), (100, 16384), (40, 16448), (300, 18944), (33, 24576)])
def test_gemv_long_row_kernel_options(kq, n, k):
    """The long-row kernel (4096 < k <= 24576; 12 waves per block beyond 16384) at every rows-per-block / row-group setting: each matches the
    oracle, and all give the same bits (one chunk per lane and a fixed reduction order in every setting)."""
    s = synth()
    case(f"gemv long rows n={n} k={k}, rows per block 4/8/16 x row groups 1/2")
    wq = s.q4_weight(n, k, 500 + n)
    x = s.bf16_normal((1, k), 501 + n)
    want = O.q4_matmul(O.Q4Planar(*wq), x)[0]
    w, xd = q4_dev(kq, wq), dev_bf16(x)
    outs = {}
    try:
        for groups in (1, 2):
            for rows in (4, 8, 16):
                kq.set_option(kq.OPT_GEMV_LONG_ROWS, rows)
                kq.set_option(kq.OPT_GEMV_LONG_GROUPS, groups)
                outs[(groups, rows)] = kq.q4_linear(w, xd, out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
    finally:
        kq.set_option(kq.OPT_GEMV_LONG_ROWS, 4)
        kq.set_option(kq.OPT_GEMV_LONG_GROUPS, 1)
    for key, y in outs.items():
        assert_rms_close(y, want, what=f"groups={key[0]} rows={key[1]}")
        assert np.array_equal(y.view(np.uint32), outs[(1, 4)].view(np.uint32)), key


@pytest.mark.parametrize("epi", ["f32", "bf16", "acc_f32", "acc_bf16"])
def test_gemv_longest_rows_epilogues(kq, epi):
    """m = 1 over k = 18944 (a 7B-class down projection, 592 chunks: the 12-wave long-row blocks) with every
    epilogue, against the oracle."""
    s = synth()
    n, k = 3584, 18944
    case(f"gemv n={n} k={k} epilogue {epi}")
    wq = s.q4_weight(n, k, 610)
    x = s.bf16_normal((1, k), 611)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    w, xd = q4_dev(kq, wq), dev_bf16(x)
    if epi == "f32":
        assert_rms_close(kq.q4_linear(w, xd, out_dtype=kq.DTYPE_F32).cpu().numpy(), want, what=epi)
    elif epi == "bf16":
        yb = kq.q4_linear(w, xd, out_dtype=kq.DTYPE_BF16)
        assert_bf16_rounded_close(host_bits(yb), want, rms(want), what=epi)
    elif epi == "acc_f32":
        base = s.f32_normal((1, n), 612)
        acc = torch.from_numpy(base.copy()).cuda()
        kq.q4_linear(w, xd, y=acc, accumulate=True)
        assert_rms_close(acc.cpu().numpy() - base, want, what=epi)
    else:
        base_b = s.bf16_normal((1, n), 613)
        acc = dev_bf16(base_b).clone()
        kq.q4_linear(w, xd, y=acc, accumulate=True)
        assert_bf16_rounded_close(host_bits(acc), O.bf16_to_f32(base_b) + want, rms(want), what=epi)


def test_stream_read_reads_every_piece(kq):
    """The streaming-floor helper reads every byte: hits[i] = 1 exactly for the 1 KB pieces holding a
    16-byte unit whose four words xor to `match` (a ragged last piece included)."""
    case("stream_read 37 x 1 KB + 48 B, three planted units")
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2 ** 32, size=(37 * 1024 + 48) // 4, dtype=np.uint32)
    match = 0x2545F491
    for unit in (3, 20 * 64 + 63, 37 * 64 + 2):  # make these units xor to `match` through their first word
        u = words[4 * unit:4 * unit + 4]
        u[0] ^= np.bitwise_xor.reduce(u) ^ np.uint32(match)
    unit_hit = np.bitwise_xor.reduce(words.reshape(-1, 4), axis=1) == np.uint32(match)
    want = np.zeros(38, dtype=bool)
    np.logical_or.at(want, np.arange(unit_hit.size) // 64, unit_hit)
    buf = torch.from_numpy(words.view(np.int32)).cuda()
    hits = kq.stream_read(buf, match=match).cpu().numpy()
    assert hits.size == 38
    assert np.array_equal(hits != 0, want) and hits[[0, 20, 37]].all()
    with pytest.raises(kq.KrError):
        kq.stream_read(buf[:3])  # 12 bytes: not a multiple of 16


def test_gemv_accumulate_modes(kq):
    s = synth()
    case("gemv accumulate f32 and bf16 (cfg1 down shape 2048x11008)")
    wq = s.q4_weight(2048, 11008, 1003)
    x = s.bf16_normal((1, 11008), 7)
    r0 = s.bf16_normal((1, 2048), 8)
    w = q4_dev(kq, wq)
    y = O.q4_matmul(O.Q4Planar(*wq), x)[0]
    # f32 residual: res += y
    res32 = torch.from_numpy(O.bf16_to_f32(r0)).cuda()
    kq.q4_linear(w, dev_bf16(x), y=res32, accumulate=True)
    assert_rms_close(res32.cpu().numpy()[0] - O.bf16_to_f32(r0)[0], y, what="acc f32")
    # bf16 residual in place: res = bf16(f32(res) + y)
    res16 = dev_bf16(r0).clone()
    kq.encode_q4_linear_accumulate(w, dev_bf16(x), res16, 2048, 11008)
    want = O.bf16_to_f32(r0)[0] + y
    assert_bf16_rounded_close(host_bits(res16)[0], want, rms(y), what="acc bf16")


def test_gemv_grid_invariance_and_determinism(kq):
    case("gemv persistent grid (4 blocks) vs full grid, bitwise; 3 repeated runs")
    w = q4_dev(kq, (FIX["persist_256_qw"], FIX["persist_256_sc"], FIX["persist_256_bi"]))
    x = dev_bf16(FIX["persist_256_x"])
    full = host_bits(kq.q4_linear(w, x, out_dtype=kq.DTYPE_BF16))
    kq.set_option(kq.OPT_GEMV_MAX_BLOCKS, 4)
    try:
        small = host_bits(kq.q4_linear(w, x, out_dtype=kq.DTYPE_BF16))
    finally:
        kq.set_option(kq.OPT_GEMV_MAX_BLOCKS, 0)
    assert np.array_equal(full, small)
    s = synth()
    wq = s.q4_weight(11008, 2048, 0)
    xb = dev_bf16(s.bf16_normal((1, 2048), 1))
    wd = q4_dev(kq, wq)
    runs = [kq.q4_linear(wd, xb, out_dtype=kq.DTYPE_F32).cpu().numpy() for _ in range(3)]
    assert all(np.array_equal(runs[0].view(np.uint32), r.view(np.uint32)) for r in runs[1:])


def test_gemv_multi_token_rows(kq):
    s = synth()
    case("linear m=3, k=2048, n=1000")
    wq = s.q4_weight(1000, 2048, 31)
    x = s.bf16_normal((3, 2048), 32)
    y = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, O.q4_matmul(O.Q4Planar(*wq), x), what="m=3")


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("n,k", [(1000, 2048), (37, 128), (129, 1408), (300, 11008), (77, 4160)])
def test_gemv_tokens_linear(kq, m, n, k):
    """2 <= m <= 4 on the GEMV kernels (k <= 2048: wave kernel; longer rows: the long-row kernel):
    all four epilogues against the oracle, and against the few-token MFMA kernel."""
    s = synth()
    case(f"linear tokens m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 40 + m)
    x = s.bf16_normal((m, k), 50 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    wd, xd = q4_dev(kq, wq), dev_bf16(x)
    y = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, want, what=f"m={m} f32")
    yb = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb), want, rms(want), what=f"m={m} bf16")
    base = s.f32_normal((m, n), 60 + m)
    acc32 = torch.from_numpy(base.copy()).cuda()
    kq.q4_linear(wd, xd, y=acc32, accumulate=True)
    assert_rms_close(acc32.cpu().numpy() - base, want, what=f"m={m} acc f32")
    base_b = s.bf16_normal((m, n), 70 + m)
    accb = dev_bf16(base_b).clone()
    kq.q4_linear(wd, xd, y=accb, accumulate=True)
    assert_bf16_rounded_close(host_bits(accb), O.bf16_to_f32(base_b) + want, rms(want), what=f"m={m} acc bf16")
    if k <= 2048:  # the MFMA few-token kernel covers one 2048-column slab without a workspace
        kq.set_option(kq.OPT_GEMV_TOKENS, 0)  # raises on failure
        assert kq.get_option(kq.OPT_GEMV_TOKENS) == 0
        try:
            y2 = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_F32).cpu().numpy()
        finally:
            kq.set_option(kq.OPT_GEMV_TOKENS, 1)
        assert np.max(np.abs(y - y2)) <= 1e-4 * rms(want)


@pytest.mark.parametrize("m", [5, 8, 13, 16])
@pytest.mark.parametrize("n,k", [(300, 11008), (77, 4160)])
def test_linear_few_tokens_long_k(kq, m, n, k):
    """5 <= m <= 16 tokens over k > 2048 without a workspace (kr_q4_linear has none for the few-token
    kernel's split K): the token GEMV in chunks of at most 4 tokens.  All four epilogues against the
    oracle; every token's row as a call with that token alone gives it (bit for bit)."""
    s = synth()
    case(f"linear few tokens long k m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 140 + m)
    x = s.bf16_normal((m, k), 150 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    wd, xd = q4_dev(kq, wq), dev_bf16(x)
    y = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_F32)
    assert_rms_close(y.cpu().numpy(), want, what=f"m={m} f32")
    for t in (0, m // 2, m - 1):
        yt = kq.q4_linear(wd, xd[t:t + 1].contiguous(), out_dtype=kq.DTYPE_F32)
        assert torch.equal(yt[0].view(torch.int32), y[t].view(torch.int32)), f"token {t}"
    yb = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb), want, rms(want), what=f"m={m} bf16")
    base = s.f32_normal((m, n), 160 + m)
    acc32 = torch.from_numpy(base.copy()).cuda()
    kq.q4_linear(wd, xd, y=acc32, accumulate=True)
    assert_rms_close(acc32.cpu().numpy() - base, want, what=f"m={m} acc f32")
    base_b = s.bf16_normal((m, n), 170 + m)
    accb = dev_bf16(base_b).clone()
    kq.q4_linear(wd, xd, y=accb, accumulate=True)
    assert_bf16_rounded_close(host_bits(accb), O.bf16_to_f32(base_b) + want, rms(want), what=f"m={m} acc bf16")


WS_BIG = {}


@pytest.mark.parametrize("m", [2, 5, 16, 17, 40, 63, 64, 96])
@pytest.mark.parametrize("n,k", [(2048, 11008), (300, 4160), (2048, 2752), (96, 2112)])
def test_linear_ws_long_k(kq, m, n, k):
    """kr_q4_linear_ws: the same linear with a caller workspace, so that K splits over blocks (the
    few-token kernel's in-launch reduction at 5 <= m <= 63, the tiled kernel's split and reduction launch
    at m >= 64).  f32 and bf16-accumulate outputs against the oracle, the same bits on a second call,
    the workspace's counters left at zero, and one workspace sized for 96 rows serving every m."""
    s = synth()
    case(f"linear with workspace m={m} n={n} k={k}")
    wq = s.q4_weight(n, k, 180 + m + n)
    x = s.bf16_normal((m, k), 190 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    wd, xd = q4_dev(kq, wq), dev_bf16(x)
    ws = kq.linear_workspace(m, n, k)
    y = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_F32, workspace=ws)
    assert_rms_close(y.cpu().numpy(), want, what=f"m={m} f32")
    assert int(torch.count_nonzero(ws[:2048])) == 0
    y2 = kq.q4_linear(wd, xd, out_dtype=kq.DTYPE_F32, workspace=ws)
    assert torch.equal(y2.view(torch.int32), y.view(torch.int32))
    if (n, k) not in WS_BIG:
        WS_BIG[(n, k)] = kq.linear_workspace(96, n, k)
    base_b = s.bf16_normal((m, n), 200 + m)
    accb = dev_bf16(base_b).clone()
    kq.q4_linear(wd, xd, y=accb, accumulate=True, workspace=WS_BIG[(n, k)])
    assert_bf16_rounded_close(host_bits(accb), O.bf16_to_f32(base_b) + want, rms(want), what=f"m={m} acc bf16")
    assert int(torch.count_nonzero(WS_BIG[(n, k)][:2048])) == 0


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("n,k", [(500, 2048), (37, 1408), (11008, 2048)])
def test_gemv_tokens_gate_up(kq, m, n, k):
    s = synth()
    case(f"gate_up tokens m={m} n={n} k={k}")
    g, u = s.q4_weight(n, k, 80 + m), s.q4_weight(n, k, 90 + m)
    x = s.bf16_normal((m, k), 100 + m)
    want = O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x)
    a = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(a, want, what=f"gate_up m={m}")


# ---------------------------------------------------------------- gate+up+act and MLP

@pytest.mark.parametrize("name", ["swiglu_9x128", "swiglu_11x128"])
def test_gate_up_reference_fixtures(kq, name):
    case(f"gate_up fixture {name}")
    g = q4_dev(kq, (FIX[f"{name}_gqw"], FIX[f"{name}_gsc"], FIX[f"{name}_gbi"]))
    u = q4_dev(kq, (FIX[f"{name}_uqw"], FIX[f"{name}_usc"], FIX[f"{name}_ubi"]))
    x = dev_bf16(FIX[f"{name}_x"])
    want = FIX[f"{name}_a"]
    a = kq.gate_up_act(g, u, x, out_dtype=kq.DTYPE_F32).cpu().numpy()[0]
    assert np.max(np.abs(a - want)) < 0.05
    assert_rms_close(a, want, what=name)
    ab = kq.gate_up_act(g, u, x, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(ab)[0], want, rms(want), what=name)


@pytest.mark.parametrize("act", [0, 1, 2])
def test_gate_up_config1_shapes(kq, act):
    s = synth()
    case(f"gate_up cfg1 11008x2048 act={act}")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    x = s.bf16_normal((1, 2048), 1004)
    a = kq.gate_up_act(q4_dev(kq, g), q4_dev(kq, u), dev_bf16(x), out_dtype=kq.DTYPE_F32,
                       activation=act).cpu().numpy()
    want = O.q4_gate_up_act(O.Q4Planar(*g), O.Q4Planar(*u), x, variant=act)
    assert_rms_close(a, want, what=f"gate_up act={act}")


@pytest.mark.parametrize("B", [1, 4, 16])
def test_mlp_config1(kq, B):
    s = synth()
    case(f"mlp cfg1 B={B}: h += down(silu(gate h) * up h), h bf16 in place")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    d = s.q4_weight(2048, 11008, 1003)
    h0 = s.bf16_normal((B, 2048), 1010 + B)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    h = dev_bf16(h0).clone()
    kq.mlp(G, U, D, h)
    want = O.bf16_to_f32(h0) + delta
    # the bf16 intermediate may round differently from the oracle's where g, u differ in the last
    # f32 bits; those flips move the output by up to ~1e-3 of its RMS, so this check uses the 1e-2 bar
    assert_bf16_rounded_close(host_bits(h), want, rms(delta), rel=1e-2, what=f"mlp B={B} bf16 residual")
    # f32 residual stream: exposes the MLP output itself to the RMS bar
    h32 = torch.from_numpy(O.bf16_to_f32(h0)).cuda()
    kq.mlp(G, U, D, h32, x=dev_bf16(h0))
    got = h32.cpu().numpy() - O.bf16_to_f32(h0)
    err = assert_rms_close(got, delta, what=f"mlp B={B}")
    delta32 = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0, bf16_intermediate=False)
    print(f"mlp B={B}: max err vs oracle {err / rms(delta):.2e} of rms; vs f32-intermediate oracle "
          f"{np.max(np.abs(got - delta32)) / rms(delta32):.2e} of rms")
    assert_rms_close(got, delta32, what=f"mlp B={B} vs f32 intermediate")


@pytest.mark.parametrize("m", [5, 9, 16])
def test_mlp_split_k_in_launch_reduction(kq, m):
    """Few-token MLP: the down projection's K split (11008 = 6 slabs of 2048) reduced by the last block of
    each run gives the bits of the separate reduction launch (same slab order); every call leaves the
    workspace's counters at zero; graph replays give the eager bits."""
    s = synth()
    case(f"mlp m={m}: split-K reduced in launch vs second launch, counters, 3 graph replays")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    d = s.q4_weight(2048, 11008, 1003)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    h0 = s.bf16_normal((m, 2048), 1200 + m)
    x = dev_bf16(h0)
    ws = kq.mlp_workspace(m, 2048, 11008)
    tickets = ws[:2048]  # the first 512 words of the workspace
    outs = {}
    try:
        for tk in (0, 1, 1):
            kq.set_option(kq.OPT_SPLITK_TICKETS, tk)
            h = torch.zeros((m, 2048), dtype=torch.float32, device="cuda")
            kq.mlp(G, U, D, h, x=x, workspace=ws)
            outs.setdefault(tk, []).append(h.cpu().numpy())
            assert int(torch.count_nonzero(tickets)) == 0
    finally:
        kq.set_option(kq.OPT_SPLITK_TICKETS, 1)
    for got in outs[1]:
        assert np.array_equal(got.view(np.uint32), outs[0][0].view(np.uint32))
    # a workspace sized for 16 rows serves smaller m too (the counters sit at the same place for every m)
    big = kq.mlp_workspace(16, 2048, 11008)
    for mm in (16, m):
        hh = torch.zeros((mm, 2048), dtype=torch.float32, device="cuda")
        kq.mlp(G, U, D, hh, x=x[:mm] if mm <= m else dev_bf16(s.bf16_normal((mm, 2048), 1300)), workspace=big)
        assert int(torch.count_nonzero(big[:2048])) == 0
    assert np.array_equal(hh.cpu().numpy().view(np.uint32), outs[0][0].view(np.uint32))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    assert_rms_close(outs[1][0], delta, what=f"mlp m={m} (in-launch split-K reduction)")
    h = torch.zeros((m, 2048), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            kq.mlp(G, U, D, h, x=x, workspace=ws)
    torch.cuda.synchronize()
    for i in range(3):
        h.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(h.cpu().numpy().view(np.uint32), outs[0][0].view(np.uint32)), f"replay {i}"
        assert int(torch.count_nonzero(tickets)) == 0


@pytest.mark.parametrize("m,inter", [(9, 16384), (12, 20480)])
def test_mlp_split_k_edges(kq, m, inter):
    """The down projection's K split at its edges: 16384 = 8 slabs (the most the in-launch reduction takes)
    and 20480 = 10 slabs (reduced by a second launch); both against the oracle, and option on/off give the
    same bits."""
    s = synth()
    case(f"mlp m={m} hidden=512 inter={inter}: split-K edges")
    g, u = s.q4_weight(inter, 512, 1401), s.q4_weight(inter, 512, 1402)
    d = s.q4_weight(512, inter, 1403)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    h0 = s.bf16_normal((m, 512), 1404)
    x = dev_bf16(h0)
    ws = kq.mlp_workspace(m, 512, inter)
    outs = []
    try:
        for tk in (1, 0):
            kq.set_option(kq.OPT_SPLITK_TICKETS, tk)
            h = torch.zeros((m, 512), dtype=torch.float32, device="cuda")
            kq.mlp(G, U, D, h, x=x, workspace=ws)
            outs.append(h.cpu().numpy())
            assert int(torch.count_nonzero(ws[:2048])) == 0
    finally:
        kq.set_option(kq.OPT_SPLITK_TICKETS, 1)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    assert_rms_close(outs[0], delta, what=f"mlp m={m} inter={inter}")


@pytest.mark.parametrize("m", [1, 3, 16])
def test_linear_at_the_k_limit(kq, m):
    """k = 24576, the documented maximum: the m = 1 split-K block kernel, the token GEMV and the few-token
    kernel (12 slabs, through the MFMA path's workspace-free fallback or its own split) against the oracle."""
    s = synth()
    case(f"q4_linear m={m} n=96 k=24576")
    wq = s.q4_weight(96, 24576, 1500 + m)
    x = s.bf16_normal((m, 24576), 1501)
    y = kq.q4_linear(q4_dev(kq, wq), dev_bf16(x), out_dtype=kq.DTYPE_F32).cpu().numpy()
    assert_rms_close(y, O.q4_matmul(O.Q4Planar(*wq), x), what=f"k limit m={m}")


# ---------------------------------------------------------------- MLP (m == 1): shapes, reuse, graphs

@pytest.mark.parametrize("hidden,inter", [(2048, 11008), (256, 384), (512, 1408), (1024, 4096)])
def test_mlp_m1_shapes_and_workspace_reuse(kq, hidden, inter):
    s = synth()
    case(f"mlp m=1 hidden={hidden} inter={inter}: 3 calls on one workspace, f32 residual")
    g, u = s.q4_weight(inter, hidden, 21), s.q4_weight(inter, hidden, 22)
    d = s.q4_weight(hidden, inter, 23)
    h0 = s.bf16_normal((1, hidden), 24)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    ws = kq.mlp_workspace(1, hidden, inter)
    h32 = torch.from_numpy(O.bf16_to_f32(h0)).cuda()
    x = dev_bf16(h0)
    outs = []
    for _ in range(3):
        kq.mlp(G, U, D, h32, x=x, workspace=ws)
        outs.append(h32.cpu().numpy().copy())
    base = O.bf16_to_f32(h0)
    assert_rms_close(outs[0] - base, delta, what="call 1")
    assert_rms_close(outs[2] - outs[1], delta, rel=2e-2, what="call 3")  # f32 residual rounding grows


def test_mlp_bf16_in_place_and_determinism(kq):
    s = synth()
    case("mlp m=1 cfg1, bf16 h in place (x = h), 2 runs bitwise equal")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    d = s.q4_weight(2048, 11008, 1003)
    h0 = s.bf16_normal((1, 2048), 1011)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    runs = []
    for _ in range(2):
        h = dev_bf16(h0).clone()
        kq.mlp(G, U, D, h)
        runs.append(host_bits(h))
    assert np.array_equal(runs[0], runs[1])
    assert_bf16_rounded_close(runs[0], O.bf16_to_f32(h0) + delta, rms(delta), what="bf16 in place")


def test_mlp_graph_replays(kq):
    s = synth()
    case("mlp m=1 captured in a HIP graph, 3 replays vs eager")
    g, u = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002)
    d = s.q4_weight(2048, 11008, 1003)
    h0 = s.bf16_normal((1, 2048), 1011)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    ws = kq.mlp_workspace(1, 2048, 11008)
    x = dev_bf16(h0)
    h = torch.zeros((1, 2048), dtype=torch.float32, device="cuda")
    kq.mlp(G, U, D, h, x=x, workspace=ws)
    eager = h.cpu().numpy().copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        h.zero_()
        with torch.cuda.graph(graph, stream=stream):
            kq.mlp(G, U, D, h, x=x, workspace=ws)
    torch.cuda.synchronize()
    for i in range(3):
        h.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(h.cpu().numpy().view(np.uint32), eager.view(np.uint32)), f"replay {i}"


@pytest.mark.parametrize("m", [16, 96])
def test_linear_ws_graph_replays(kq, m):
    """kr_q4_linear_ws captured in a HIP graph (the split-K partials and counters in the workspace):
    3 replays, with eager work on the same workspace between them, each giving the eager bits."""
    s = synth()
    case(f"linear_ws m={m} in a HIP graph, 3 replays vs eager")
    n, k = 2048, 11008
    wq = s.q4_weight(n, k, 1003)
    x = dev_bf16(s.bf16_normal((m, k), 1020 + m))
    W = q4_dev(kq, wq)
    ws = kq.linear_workspace(m, n, k)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    kq.q4_linear(W, x, y=y, workspace=ws)
    eager = y.cpu().numpy().copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            kq.q4_linear(W, x, y=y, workspace=ws)
    torch.cuda.synchronize()
    for i in range(3):
        y.zero_()
        other = kq.q4_linear(W, x, out_dtype=kq.DTYPE_F32, workspace=ws)  # eager use of the workspace
        torch.cuda.synchronize()
        assert np.array_equal(other.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), eager.view(np.uint32)), f"replay {i}"
        assert int(torch.count_nonzero(ws[:2048])) == 0
