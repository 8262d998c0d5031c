"""kr_q4_mlp_noalloc (the MLP with the library's per-GPU scratch array as its workspace) against
kr_q4_mlp with a caller workspace, through the C ABI: identical bits (the same kernels run on the
same inputs), on consecutive calls whose second one is smaller, so the second call finds the
array holding the first call's contents."""
import numpy as np
import pytest
import torch

import oracle as O
from _util import assert_rms_close, dev_bf16, q4_dev

pytestmark = pytest.mark.gpu

H, I = 2048, 11008


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def mats(kq):
    from kriya_q4 import synth
    return [q4_dev(kq, synth.q4_weight(n, k, 7100 + i)) for i, (n, k) in enumerate(((I, H), (I, H), (H, I)))]


@pytest.mark.parametrize("ms", [(16, 5), (3, 1), (37, 9)])
def test_noalloc_mlp_matches_workspace_mlp(kq, mats, ms):
    from kriya_q4 import synth
    g, u, d = mats
    for i, m in enumerate(ms):
        case(f"mlp_noalloc call {i} m={m} (sequence {ms})")
        h0 = synth.bf16_normal((m, H), 7200 + m)
        want = dev_bf16(h0).clone()
        kq.mlp(g, u, d, want, workspace=kq.mlp_workspace(m, H, I))
        got = dev_bf16(h0).clone()
        kq.mlp_noalloc(g, u, d, got)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"m={m}"


def test_noalloc_mlp_f32_residual_vs_oracle(kq, mats):
    """h f32 with a separate bf16 input x, against the oracle's MLP (the tolerance of every matmul)."""
    from kriya_q4 import synth
    g, u, d = mats
    m = 4
    case(f"mlp_noalloc f32 residual m={m} vs oracle")
    x = synth.bf16_normal((m, H), 7301)
    h0 = np.random.default_rng(7302).standard_normal((m, H)).astype(np.float32)
    h = torch.from_numpy(h0).cuda()
    kq.mlp_noalloc(g, u, d, h, x=dev_bf16(x))
    planars = [O.Q4Planar(w.qw.cpu().numpy().view(np.uint32), w.scales.cpu().numpy().view(np.uint16),
                          w.biases.cpu().numpy().view(np.uint16)) for w in (g, u, d)]
    delta = O.q4_mlp(*planars, x)
    assert_rms_close(h.cpu().numpy() - h0, delta, what="noalloc f32")


def test_noalloc_rejects_sizes_beyond_its_scratch(kq, mats):
    g, u, d = mats
    case("mlp_noalloc m=64 exceeds the scratch: KR_E_WORKSPACE, nothing enqueued")
    assert kq.lib().kr_q4_mlp_noalloc_max_bytes() == 4 << 20
    assert kq.mlp_workspace_bytes(64, H, I) > 4 << 20
    h = torch.zeros((64, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(kq.KrError) as ei:
        kq.mlp_noalloc(g, u, d, h)
    assert ei.value.code == kq.KR_E_WORKSPACE
    assert int(h.view(torch.int16).abs().sum().item()) == 0
