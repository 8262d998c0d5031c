"""One GPU's share of the config 1 MLP under 4-way tensor parallelism, at its real shapes.

gate/up split by output rows (column-parallel: gate/up [2752, 2048], bound as row views of the full planar
triplet, no copy), down split over K in whole 64-groups (row-parallel: down [2048, 2752], the column slice a
sharded checkpoint loader would hand each GPU).  Each share writes an f32 partial [B, 2048]; the all-reduce
sums the four.  Here the four shares run one after the other on the one GPU and their partials are summed on
the host in shard order: every share is checked against the oracle on its own weights, and the sum against
the oracle's unsharded MLP.  (Reference: the dense MLP, encoder.rs:2851-2906; 11008 = 64 * 4 * 43, so the
down projection shards over whole groups only for TP in {1, 2, 4}.)
"""
import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_rms_close, dev_bf16, q4_dev, rms

pytestmark = pytest.mark.gpu
TP = 4


def case(msg):
    print(f"[case] {msg}", flush=True)


def k_columns(p, lo, hi):
    """Columns [lo, hi) of a planar triplet (lo, hi multiples of 64), contiguous."""
    qw, sc, bi = p
    return (np.ascontiguousarray(qw[:, lo // 8:hi // 8]), np.ascontiguousarray(sc[:, lo // 64:hi // 64]),
            np.ascontiguousarray(bi[:, lo // 64:hi // 64]))


@pytest.mark.parametrize("B", [1, 16])
def test_tp4_shares(kq, B):
    from kriya_q4 import synth as s

    H, I = 2048, 11008
    Is = I // TP
    case(f"cfg1 MLP B={B}, TP={TP} shares: gate/up [{Is},{H}] row views, down [{H},{Is}] K columns")
    g, u, d = s.q4_weight(I, H, 1001), s.q4_weight(I, H, 1002), s.q4_weight(H, I, 1003)
    h0 = s.bf16_normal((B, H), 1010 + B)
    G, U = q4_dev(kq, g), q4_dev(kq, u)
    x = dev_bf16(h0)
    parts = []
    for sh in range(TP):
        lo, hi = sh * Is, (sh + 1) * Is
        Gs, Us = G.rows(lo, hi), U.rows(lo, hi)  # views into the full matrices
        dp = k_columns(d, lo, hi)
        Ds = q4_dev(kq, dp)
        part = torch.zeros((B, H), dtype=torch.float32, device="cuda")
        kq.mlp(Gs, Us, Ds, part, x=x)
        got = part.cpu().numpy()
        gp = O.Q4Planar(*g).rows(lo, hi)
        up = O.Q4Planar(*u).rows(lo, hi)
        want = O.q4_mlp(gp, up, O.Q4Planar(*dp), h0)
        assert_rms_close(got, want, what=f"TP share {sh} B={B}")
        parts.append(got)
    total = parts[0]
    for p in parts[1:]:
        total = total + p  # the all-reduce's sum, in shard order
    full = O.q4_mlp(O.Q4Planar(*g), O.Q4Planar(*u), O.Q4Planar(*d), h0)
    err = assert_rms_close(total, full, what=f"TP={TP} sum vs unsharded B={B}")
    # and against this library's own unsharded MLP on the same GPU
    h32 = torch.zeros((B, H), dtype=torch.float32, device="cuda")
    kq.mlp(G, U, q4_dev(kq, d), h32, x=x)
    assert_rms_close(total, h32.cpu().numpy(), what=f"TP={TP} sum vs the one-GPU MLP B={B}")
    print(f"TP={TP} B={B}: sum of shares vs oracle {err / rms(full):.2e} of rms")
