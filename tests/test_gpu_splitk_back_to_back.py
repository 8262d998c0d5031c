"""Split-K reductions inside the launch, under calls queued back to back on one stream.

The few-token down projection over K = 11008 splits K over 6 slabs; the blocks of a run publish
f32 partials into the caller's workspace and the last block to take the run's ticket sums them in
slab order.  The partials go through device-coherent stores and loads.  Each call here reuses the
same workspace with a different input, with no host synchronisation between calls.  A reducer that
read a stale partial (an earlier call's, or a line cached by another XCD's L2) would produce bits
different from those of the separate reduction launch (KR_OPT_SPLITK_TICKETS = 0), which is ordered
by the stream.  The same check runs kr_q4_linear_ws over the TP = 4 share's down projection
(K = 2752, 43 groups: two slabs, the second of odd length).  Distinct inputs give distinct outputs,
so stale data cannot pass unnoticed.  (Reference: the dense MLP and linear entry points,
encoder.rs:2361-2420, 2851-2906; its split-K has no counterpart, so the fallback launch is the bar.)
"""
import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_rms_close, dev_bf16, q4_dev

pytestmark = pytest.mark.gpu

CALLS = 24


def synth():
    from kriya_q4 import synth as s
    return s


def case(msg):
    print(f"[case] {msg}", flush=True)


def _runs(kq, enqueue, nout):
    """Outputs of CALLS queued calls, with the in-launch reduction off, on, and on again."""
    res = {}
    try:
        for label, tk in (("launch", 0), ("ticket", 1), ("ticket2", 1)):
            kq.set_option(kq.OPT_SPLITK_TICKETS, tk)
            outs = [torch.zeros(nout, dtype=torch.float32, device="cuda") for _ in range(CALLS)]
            for i, o in enumerate(outs):
                enqueue(i, o)
            torch.cuda.synchronize()
            res[label] = [o.cpu().numpy() for o in outs]
    finally:
        kq.set_option(kq.OPT_SPLITK_TICKETS, 1)
    return res


def _check(res, what):
    for i in range(CALLS):
        for label in ("ticket", "ticket2"):
            assert np.array_equal(res[label][i].view(np.uint32), res["launch"][i].view(np.uint32)), \
                f"{what}: call {i} ({label}) differs from the reduction launch"
    assert not np.array_equal(res["launch"][0], res["launch"][1]), f"{what}: inputs must differ"


@pytest.mark.parametrize("m", [8, 16])
def test_mlp_tickets_back_to_back(kq, m):
    s = synth()
    case(f"mlp m={m}: {CALLS} queued calls on one workspace, in-launch reduction vs second launch")
    g, u, d = s.q4_weight(11008, 2048, 1001), s.q4_weight(11008, 2048, 1002), s.q4_weight(2048, 11008, 1003)
    G, U, D = (q4_dev(kq, t) for t in (g, u, d))
    xs_host = [s.bf16_normal((m, 2048), 1600 + i) for i in range(CALLS)]
    xs = [dev_bf16(x) for x in xs_host]
    ws = kq.mlp_workspace(m, 2048, 11008)

    def enqueue(i, out):
        kq.mlp(G, U, D, out.view(m, 2048), x=xs[i], workspace=ws)

    res = _runs(kq, enqueue, m * 2048)
    _check(res, f"mlp m={m}")
    assert int(torch.count_nonzero(ws[:2048])) == 0
    last = CALLS - 1
    delta = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), xs_host[last])
    assert_rms_close(res["ticket"][last].reshape(m, 2048), delta, what=f"mlp m={m} call {last}")


@pytest.mark.parametrize("m", [6, 16])
def test_linear_ws_tickets_back_to_back(kq, m):
    s = synth()
    case(f"linear_ws m={m} [2048, 2752]: {CALLS} queued calls on one workspace")
    wq = s.q4_weight(2048, 2752, 1700)
    W = q4_dev(kq, wq)
    xs_host = [s.bf16_normal((m, 2752), 1710 + i) for i in range(CALLS)]
    xs = [dev_bf16(x) for x in xs_host]
    ws = kq.linear_workspace(m, 2048, 2752)

    def enqueue(i, out):
        kq.q4_linear(W, xs[i], y=out.view(m, 2048), out_dtype=kq.DTYPE_F32, workspace=ws)

    res = _runs(kq, enqueue, m * 2048)
    _check(res, f"linear_ws m={m}")
    assert int(torch.count_nonzero(ws[:2048])) == 0
    want = O.q4_matmul(O.Q4Planar(*wq), xs_host[0])
    assert_rms_close(res["ticket"][0].reshape(m, 2048), want, what=f"linear_ws m={m} call 0")
