"""GPU parity of the MoE path (config 4) against the CPU oracle and the
reference's own scan/scatter known answers.

  routing  : experts, counts, offsets and the sorted assignment list are
             integers and must match exactly; weights within 2e-6 relative
             (the device expf/divide are not the host's).
  experts  : max |gpu - oracle| <= 1e-2 * RMS(oracle) on f32 outputs.
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
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


def i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.uint32)).view(np.int32)).cuda()


def u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


def check_route(r, experts, weights, counts, offsets, sorted_assign):
    assert np.array_equal(u32(r.selected).ravel(), experts.ravel())
    assert np.array_equal(u32(r.counts), counts)
    assert np.array_equal(u32(r.offsets), offsets)
    assert np.array_equal(u32(r.sorted_assign)[: experts.size], sorted_assign)
    np.testing.assert_allclose(r.weights.cpu().numpy(), weights, rtol=2e-6, atol=0)


@pytest.mark.parametrize("idx", range(3))
def test_scan_scatter_reference_kats(kq, idx):
    """test_shader_compile.rs:2988-3117 expectations for E in {8, 64, 256}."""
    kat = KATS["moe_scan_scatter"][idx]
    case(f"scan/scatter KAT E={kat['E']} T={kat['T']} K={kat['K']}")
    counts, offsets, scatter = kq.moe_scan_scatter(i32(kat["experts"]), kat["E"])
    assert u32(offsets).tolist() == kat["offsets"]
    assert u32(scatter).tolist() == kat["scatter"]
    assert u32(counts).tolist() == list(np.diff(kat["offsets"]))
    # the slot of assignment a inside its bucket
    pos = {a: i for i, a in enumerate(kat["scatter"])}
    slots = [pos[a] - kat["offsets"][e] for a, e in enumerate(kat["experts"])]
    assert slots == kat["slots"]


def test_scan_scatter_out_of_range_id(kq):
    case("scan/scatter with an id >= E")
    sel = np.array([1, 0, 9, 1, 2], np.uint32)
    counts, offsets, scatter = kq.moe_scan_scatter(i32(sel), 4)
    assert u32(offsets).tolist() == [0, 1, 3, 4, 4]
    assert u32(counts).tolist() == [1, 2, 1, 0]
    assert u32(scatter)[:4].tolist() == [1, 0, 3, 4]


@pytest.mark.parametrize("T,E,K,norm", [(64, 60, 4, True), (1, 60, 4, True), (33, 8, 2, False), (8, 256, 16, True),
                                        (300, 64, 1, True), (4096, 60, 4, True)])
def test_route_vs_oracle(kq, T, E, K, norm):
    s = synth()
    case(f"route T={T} E={E} K={K} normalize={norm}")
    logits = s.f32_normal((T, E), 4000 + T + E)
    want = O.moe_route(logits, K, norm)
    r = kq.moe_route(torch.from_numpy(logits).cuda(), K, norm)
    check_route(r, *want)


def test_route_ties_go_to_lower_id(kq):
    case("route ties")
    logits = np.zeros((3, 8), np.float32)
    logits[1] = [1, 3, 3, 2, 3, 0, 0, 3]
    logits[2] = [5, 5, 5, 5, 5, 5, 5, 6]
    r = kq.moe_route(torch.from_numpy(logits).cuda(), 4, True)
    sel = u32(r.selected)
    assert sel[0].tolist() == [0, 1, 2, 3]
    assert sel[1].tolist() == [1, 2, 4, 7]
    assert sel[2].tolist() == [7, 0, 1, 2]
    np.testing.assert_allclose(r.weights.cpu().numpy()[0], [0.25] * 4, rtol=1e-6)
    check_route(r, *O.moe_route(logits, 4, True))


def test_route_rejects_bad_arguments(kq):
    case("route argument checks")
    logits = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    for topk in (0, 9, 17):
        with pytest.raises(kq.KrError) as ei:
            kq.moe_route(logits, topk)
        assert ei.value.code == kq.KR_E_INVALID
    big = torch.zeros((4097, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(kq.KrError) as ei:
        kq.moe_route(big, 4)
    assert ei.value.code == kq.KR_E_SHAPE


def route_from_oracle(kq, experts, weights, counts, offsets, sorted_assign, T, E, K):
    r = kq.MoeRoute(T, E, K)
    r.selected.copy_(i32(experts).view(T, K))
    r.weights.copy_(torch.from_numpy(np.ascontiguousarray(weights)).cuda())
    r.counts.copy_(i32(counts))
    r.offsets.copy_(i32(offsets))
    r.sorted_assign[: T * K].copy_(i32(sorted_assign))
    return r


def moe_case(kq, T, E, K, hidden, inter, seed, logits=None):
    s = synth()
    g = s.q4_weight(E * inter, hidden, seed + 1)
    u = s.q4_weight(E * inter, hidden, seed + 2)
    d = s.q4_weight(E * hidden, inter, seed + 3)
    x = s.bf16_normal((T, hidden), seed + 4)
    if logits is None:
        logits = s.f32_normal((T, E), seed + 5)
    route = O.moe_route(logits, K, True)
    want = O.moe_experts(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), E, x, route[0], route[1])
    return (g, u, d, x, logits, route, want)


@pytest.mark.parametrize("T,E,K,hidden,inter", [(8, 8, 4, 128, 128), (5, 6, 2, 256, 384), (1, 16, 4, 512, 1408),
                                                (3, 5, 3, 1024, 256)])
def test_moe_experts_small(kq, T, E, K, hidden, inter):
    case(f"moe experts T={T} E={E} K={K} hidden={hidden} inter={inter}")
    g, u, d, x, logits, route, want = moe_case(kq, T, E, K, hidden, inter, 4100 + T + E)
    r = route_from_oracle(kq, *route, T, E, K)
    gd, ud, dd = q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d)
    y = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r).cpu().numpy()
    assert_rms_close(y, want, what="moe f32")
    yb = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, out_dtype=kq.DTYPE_BF16)
    assert_bf16_rounded_close(host_bits(yb), want, rms(want), rel=1e-2, what="moe bf16")
    # accumulate into a bf16 residual
    r0 = synth().bf16_normal((T, hidden), 4199)
    res = dev_bf16(r0).clone()
    kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, y=res, accumulate=True)
    assert_bf16_rounded_close(host_bits(res), O.bf16_to_f32(r0) + want, rms(want), rel=1e-2, what="moe acc")


@pytest.mark.parametrize("T,E,K,hidden,inter", [(4, 3, 2, 256, 128), (2, 60, 4, 2048, 1408), (16, 8, 1, 512, 384),
                                                (1, 60, 4, 2048, 1408)])
def test_moe_routed_gemv_and_grouped_paths(kq, T, E, K, hidden, inter):
    """Few assignments (T * K <= 16) run one GEMV per (expert, token) pair; the grouped MFMA kernel
    (KR_OPT_MOE_GEMV = 0) must give the same result to the RMS bar, both against the oracle."""
    case(f"moe routed gemv vs grouped T={T} E={E} K={K} hidden={hidden} inter={inter}")
    g, u, d, x, logits, route, want = moe_case(kq, T, E, K, hidden, inter, 4500 + T + E)
    r = route_from_oracle(kq, *route, T, E, K)
    gd, ud, dd = q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d)
    y = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r).cpu().numpy()
    assert_rms_close(y, want, what="routed gemv")
    kq.set_option(kq.OPT_MOE_GEMV, 0)
    try:
        y2 = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r).cpu().numpy()
    finally:
        kq.set_option(kq.OPT_MOE_GEMV, 1)
    assert_rms_close(y2, want, what="grouped")
    r0 = synth().bf16_normal((T, hidden), 4599)
    res = dev_bf16(r0).clone()
    kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, y=res, accumulate=True)
    assert_bf16_rounded_close(host_bits(res), O.bf16_to_f32(r0) + want, rms(want), rel=1e-2, what="routed acc")


@pytest.mark.parametrize("T", [1, 64])
def test_moe_config4(kq, T):
    """Config 4: 60 experts, top-4, hidden 2048, expert intermediate 1408, device routing."""
    E, K, H, I = 60, 4, 2048, 1408
    case(f"moe config 4 T={T}")
    g, u, d, x, logits, route, want = moe_case(kq, T, E, K, H, I, 4000)
    r = kq.moe_route(torch.from_numpy(logits).cuda(), K, True)
    check_route(r, *route)
    y = kq.moe_experts(q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d), E, dev_bf16(x), r).cpu().numpy()
    assert_rms_close(y, want, what=f"cfg4 T={T}")


def test_moe_experts_with_an_unbucketed_assignment(kq):
    """Routing from scan/scatter with an id >= E leaves offsets[E] < T * K and the tail of the sorted
    list unwritten (here: filled with 0xFFFFFFFF).  The header leaves the outputs unspecified; the
    kernels clamp the expert and the sorted entry, so the call completes with finite outputs."""
    T, E, K, H, I = 2, 4, 2, 256, 128
    case("moe experts, one assignment with an out-of-range expert id")
    s = synth()
    g, u = s.q4_weight(E * I, H, 4701), s.q4_weight(E * I, H, 4702)
    d = s.q4_weight(E * H, I, 4703)
    x = s.bf16_normal((T, H), 4704)
    sel = np.array([1, 0, 9, 3], np.uint32)
    counts, offsets, scatter = kq.moe_scan_scatter(i32(sel), E)
    assert int(offsets[E].item()) == 3
    r = kq.MoeRoute(T, E, K)
    r.selected.copy_(i32(sel).view(T, K))
    r.weights.fill_(0.5)
    r.counts.copy_(counts)
    r.offsets.copy_(offsets)
    r.sorted_assign.fill_(-1)
    r.sorted_assign[:3].copy_(scatter[:3])
    for gemv in (1, 0):
        kq.set_option(kq.OPT_MOE_GEMV, gemv)
        try:
            y = kq.moe_experts(q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d), E, dev_bf16(x), r)
            torch.cuda.synchronize()
        finally:
            kq.set_option(kq.OPT_MOE_GEMV, 1)
        assert torch.isfinite(y).all()


@pytest.mark.parametrize("T", [1, 64])
def test_moe_block_router_to_combine(kq, T):
    """Config 4 as one device stage (kr_q4_moe_block; encoder.rs:5246-5445): router Q4 GEMV with f32
    logits -> routing -> experts -> combine, against the oracle's chain.  The block's first stage is
    kr_q4_linear, whose logits are checked against the oracle's; the expected output routes on those
    device logits, so that an expert whose probability ties within f32 rounding cannot flip the
    comparison (both routings are compared too, and agree here)."""
    E, K, H, I = 60, 4, 2048, 1408
    case(f"moe block (router gemv -> route -> experts -> combine) T={T}")
    s = synth()
    router = s.q4_weight(E, H, 4801)
    g, u = s.q4_weight(E * I, H, 4802), s.q4_weight(E * I, H, 4803)
    d = s.q4_weight(E * H, I, 4804)
    x = s.bf16_normal((T, H), 4805)
    R, G, U, D = (q4_dev(kq, w) for w in (router, g, u, d))
    xd = dev_bf16(x)
    logits = kq.q4_linear(R, xd, out_dtype=kq.DTYPE_F32).cpu().numpy()
    logits_cpu = O.q4_matmul(O.Q4Planar(*router), x)
    assert_rms_close(logits, logits_cpu, what="router logits")
    route = O.moe_route(logits, K, True)
    route_cpu = O.moe_route(logits_cpu, K, True)
    assert np.array_equal(route[0], route_cpu[0])
    want = O.moe_experts(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), E, x, route[0], route[1])
    y = kq.moe_block(R, G, U, D, E, xd, K).cpu().numpy()
    assert_rms_close(y, want, what=f"moe block T={T}")
    # accumulate into a bf16 residual (the layer's h += moe(x))
    r0 = s.bf16_normal((T, H), 4806)
    res = dev_bf16(r0).clone()
    kq.moe_block(R, G, U, D, E, xd, K, y=res, accumulate=True)
    assert_bf16_rounded_close(host_bits(res), O.bf16_to_f32(r0) + want, rms(want), rel=1e-2, what="moe block acc")


def test_moe_crowded_experts(kq):
    """More than 16 tokens per expert: the 16-row chunk loop."""
    T, E, K, H, I = 40, 12, 2, 256, 128
    case("moe crowded experts (40 tokens on 2 experts)")
    logits = synth().f32_normal((T, E), 4300)
    logits[:, 3] += 20.0
    logits[:, 7] += 19.0
    g, u, d, x, logits, route, want = moe_case(kq, T, E, K, H, I, 4300, logits=logits)
    assert route[2][3] == T and route[2][7] == T
    r = kq.moe_route(torch.from_numpy(logits).cuda(), K, True)
    check_route(r, *route)
    y = kq.moe_experts(q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d), E, dev_bf16(x), r).cpu().numpy()
    assert_rms_close(y, want, what="crowded")


def test_moe_deterministic_and_graph_replay(kq):
    T, E, K, H, I = 64, 60, 4, 2048, 1408
    case("moe determinism + graph replay")
    s = synth()
    g, u, d = (q4_dev(kq, s.q4_weight(E * I, H, 4401)), q4_dev(kq, s.q4_weight(E * I, H, 4402)),
               q4_dev(kq, s.q4_weight(E * H, I, 4403)))
    x = dev_bf16(s.bf16_normal((T, H), 4404))
    logits = torch.from_numpy(s.f32_normal((T, E), 4405)).cuda()
    r = kq.MoeRoute(T, E, K)
    ws = kq.moe_workspace(T, K, H, I)
    y = torch.empty((T, H), dtype=torch.float32, device="cuda")

    def step():
        kq.moe_route(logits, K, True, out=r)
        kq.moe_experts(g, u, d, E, x, r, y=y, workspace=ws)

    step()
    torch.cuda.synchronize()
    ref = y.clone()
    step()
    assert torch.equal(y, ref)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref)


@pytest.mark.parametrize("T,E,K,hidden,inter", [(1, 60, 4, 2048, 1408), (2, 8, 2, 256, 128), (4, 6, 3, 512, 384),
                                                (16, 8, 1, 512, 384), (3, 5, 4, 128, 1024), (1, 16, 2, 2048, 2048)])
def test_moe_combine_folded_into_down_bitwise(kq, T, E, K, hidden, inter):
    """Few assignments with topk <= 4: the routed down projection sums each token's slots itself
    (KR_OPT_MOE_COMBINE = 1, the default) -- the bits of the down GEMV followed by the combine launch
    (option 0) for f32 and bf16 outputs, plain and accumulated, and within the bar of the oracle."""
    case(f"moe combine folded into down T={T} E={E} K={K} hidden={hidden} inter={inter}")
    g, u, d, x, logits, route, want = moe_case(kq, T, E, K, hidden, inter, 4800 + 7 * T + E + K)
    r = route_from_oracle(kq, *route, T, E, K)
    gd, ud, dd = q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d)
    r0 = synth().bf16_normal((T, hidden), 4899)
    outs = {}
    try:
        for opt in (0, 1):
            kq.set_option(kq.OPT_MOE_COMBINE, opt)
            yf = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r)
            yb = kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, out_dtype=kq.DTYPE_BF16)
            accf = torch.from_numpy(O.bf16_to_f32(r0)).cuda()
            kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, y=accf, accumulate=True)
            accb = dev_bf16(r0).clone()
            kq.moe_experts(gd, ud, dd, E, dev_bf16(x), r, y=accb, accumulate=True)
            outs[opt] = [t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).cpu().numpy()
                         for t in (yf, yb, accf, accb)]
    finally:
        kq.set_option(kq.OPT_MOE_COMBINE, 1)
    for i, name in enumerate(("f32", "bf16", "acc f32", "acc bf16")):
        assert np.array_equal(outs[0][i], outs[1][i]), name
    assert_rms_close(outs[1][0].view(np.float32), want, what="folded combine f32")


@pytest.mark.parametrize("E,K,hidden,inter,kind", [(60, 4, 2048, 1408, "normal"), (16, 2, 512, 384, "normal"),
                                                   (8, 8, 256, 128, "normal"), (256, 16, 128, 128, "normal"),
                                                   (12, 4, 256, 128, "ties"), (12, 6, 256, 128, "nan")])
def test_moe_route_experts_one_token_bitwise(kq, E, K, hidden, inter, kind):
    """kr_q4_moe_route_experts with one token routes inside the gate/up launch (KR_OPT_MOE_ROUTE_FUSED = 1):
    the routing arrays and y are those of the routing kernel followed by kr_q4_moe_experts (option 0) bit for
    bit -- also with tied logits (ties go to the lower id) and with NaN logits (never taken; slots left
    empty hold expert 0 with weight -inf) -- and the routing is the oracle's."""
    s = synth()
    case(f"moe route+experts one token, E={E} K={K} hidden={hidden} inter={inter} {kind}")
    g, u, d = s.q4_weight(E * inter, hidden, 4901), s.q4_weight(E * inter, hidden, 4902), s.q4_weight(E * hidden, inter, 4903)
    gd, ud, dd = q4_dev(kq, g), q4_dev(kq, u), q4_dev(kq, d)
    x = dev_bf16(s.bf16_normal((1, hidden), 4904))
    logits = s.f32_normal((1, E), 4905).astype(np.float32)
    if kind == "ties":
        logits[0, 1::3] = logits[0, 0]  # every third expert ties with expert 0
    if kind == "nan":
        logits[0, : E - 3] = np.nan  # only three finite logits for K = 6 slots
    lt = torch.from_numpy(logits).cuda()
    res = {}
    try:
        for opt in (0, 1):
            kq.set_option(kq.OPT_MOE_ROUTE_FUSED, opt)
            r = kq.MoeRoute(1, E, K)
            for t in (r.selected, r.counts, r.offsets, r.sorted_assign):
                t.fill_(-1)
            r.weights.fill_(7.0)
            y, _ = kq.moe_route_experts(gd, ud, dd, E, x, lt, K, out=r)
            res[opt] = [t.view(torch.int32).cpu().numpy() for t in (r.selected, r.weights, r.counts, r.offsets,
                                                                    r.sorted_assign, y)]
    finally:
        kq.set_option(kq.OPT_MOE_ROUTE_FUSED, 1)
    for i, name in enumerate(("selected", "weights", "counts", "offsets", "sorted", "y")):
        assert np.array_equal(res[0][i], res[1][i]), name
    want_sel, want_w, want_cnt, want_off, want_sorted = O.moe_route(logits, K, True)
    assert np.array_equal(res[1][0].ravel().astype(np.uint32), np.asarray(want_sel, np.uint32).ravel())
    assert np.array_equal(res[1][2].astype(np.uint32), np.asarray(want_cnt, np.uint32))
    assert np.array_equal(res[1][3].astype(np.uint32), np.asarray(want_off, np.uint32))
    assert np.array_equal(res[1][4].astype(np.uint32), np.asarray(want_sorted, np.uint32))
    if kind != "nan":
        want = O.moe_experts(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), E, s.bf16_normal((1, hidden), 4904),
                             want_sel, want_w)
        assert_rms_close(res[1][5].view(np.float32), want, what="route+experts")
