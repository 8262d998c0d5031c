"""The seeded input generator (kriya_q4.synth) that bench.py, smoke() and the GPU tests draw from.

SplitMix64 is pinned by its published known answers (Vigna's splitmix64.c, seed 0), the bf16 rounding by
torch's own float32 -> bfloat16 conversion, the normal draw by its moments, and the full-size inputs of
bench.py's configurations by their SHA-256 in tests/golden/input_sha256.json, so a host that regenerates
them (the GPU box, another machine) can show that it holds byte-identical inputs.
"""
import importlib.util
import json
import os

import numpy as np
import pytest

from kriya_q4 import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_splitmix64_known_answers():
    # the first outputs of SplitMix64 from state 0 (x += 0x9E3779B97F4A7C15, then the two xor-multiply rounds)
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [int(v) for v in synth.splitmix64(0, 4)] == want
    # output i of a stream does not depend on how many outputs were asked for, across the chunk edge too
    n = synth._CHUNK + 3
    long = synth.splitmix64(77, n)
    assert np.array_equal(long[:5], synth.splitmix64(77, 5))
    assert int(long[-1]) == synth.mix64((77 + n * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    f = rng.standard_normal(1 << 16).astype(np.float32) * np.float32(3.0)
    # ties: a float32 whose low 16 bits are exactly 0x8000, with even and odd bf16 mantissas
    ties = (np.arange(256, dtype=np.uint32) << np.uint32(16) | np.uint32(0x3F800000) | np.uint32(0x8000)).view(np.float32)
    f = np.concatenate([f, ties, np.array([0.0, -0.0, 1e-40, -1e-40, 3.0e38], np.float32)])
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(synth.f32_to_bf16_bits(f), want)
    assert np.array_equal(synth.bf16_bits_to_f32(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_normal_moments():
    z = synth.normal(synth.substream(9, 3), 1 << 20)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    assert abs(np.mean(np.abs(z) < 1.0) - 0.682689) < 2e-3  # P(|Z| < 1)


def test_q4_weight_layout():
    qw, s, b = synth.q4_weight(96, 256, 3)
    assert qw.shape == (96, 32) and qw.dtype == np.uint32
    assert s.shape == b.shape == (96, 4) and s.dtype == b.dtype == np.uint16
    sf, bf = synth.bf16_bits_to_f32(s), synth.bf16_bits_to_f32(b)
    assert np.all(sf >= 1e-3) and np.all(bf == -8.0 * sf)  # -8 s is exact in bf16


def _generator():
    spec = importlib.util.spec_from_file_location("make_input_hashes", os.path.join(GOLDEN, "make_input_hashes.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_full_size_inputs_match_fixture():
    with open(os.path.join(GOLDEN, "input_sha256.json")) as f:
        want = json.load(f)
    gen = _generator()
    got = {name: gen.digest(arrays) for name, arrays in gen.inputs()}
    assert sorted(got) == sorted(want)
    bad = [name for name in want if got[name] != want[name]]
    assert not bad, f"regenerated inputs differ from the fixture: {bad}"


@pytest.mark.gpu
def test_gpu_resident_inputs_match_fixture():
    """On the GPU box: every seeded input regenerated there, uploaded to HBM as bench.py uploads it and read
    back, has the fixture's SHA-256 (the bytes the timed kernels read are the ones pinned here)."""
    import hashlib

    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    with open(os.path.join(GOLDEN, "input_sha256.json")) as f:
        want = json.load(f)
    gen = _generator()
    for name, arrays in gen.inputs():
        h = hashlib.sha256()
        for a in arrays:
            dev = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8)).cuda()
            h.update(dev.cpu().numpy().tobytes())
            del dev
        assert h.hexdigest() == want[name], name
