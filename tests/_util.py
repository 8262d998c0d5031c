"""Helpers shared by the GPU parity tests."""
import numpy as np
import torch

import oracle as O


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bits (numpy) -> bf16 tensor on cuda:0."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def assert_rms_close(got, want, rel=1e-2, what=""):
    """The parity bar for floating-point outputs: max |got - want| <= rel * RMS(want)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    bound = rel * rms(want)
    assert err <= bound, f"{what}: max err {err:.4e} > {rel} * rms {rms(want):.4e}"
    return err


def assert_bf16_rounded_close(got_bits: np.ndarray, want_f32: np.ndarray, basis_rms: float, rel=1e-3, what=""):
    """bf16 outputs are RNE of an f32 value within rel * basis_rms of the oracle:
    |got - want| <= half a bf16 ulp of got (<= |got| * 2^-8) + rel * basis_rms.
    basis_rms is the RMS of the matmul result (not of a residual it is added to)."""
    got = O.bf16_to_f32(np.asarray(got_bits, np.uint16)).astype(np.float64)
    want = np.asarray(want_f32, np.float64)
    excess = np.abs(got - want) - (np.abs(got) * 2.0 ** -8 + rel * basis_rms)
    assert excess.max(initial=-1) <= 0, f"{what}: bf16 output off by {excess.max():.3e} beyond rounding"


def q4_dev(kq, planar):
    """oracle.Q4Planar or (qw, sc, bi) tuple -> device Q4Matrix."""
    if isinstance(planar, tuple):
        return kq.Q4Matrix.from_numpy(*planar)
    return kq.Q4Matrix.from_numpy(planar.qw, planar.scales, planar.biases)
