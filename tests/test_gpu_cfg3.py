"""Config 3 at its stated shape on the GPU: hidden 2048, intermediate 11008,
GQA 16/2 with head 128, vocabulary 151936 (tied Q4 embedding as the LM head),
context 512, batch 1 and 16 -- against the layer-by-layer CPU restatement
(tests/_decode_ref.py: the oracle's Q4 matmuls, f64 norms and attention,
bf16 roundings where the device stores bf16).  Reference: the decode pass
forward_and_sample_impl and its LM head (crates/kriya-backend-metal/src/
encoder.rs:4880-5516).

Bars:
- the LM head (kr_q4_linear at N = 151936) and the fused-norm few-token calls
  at H = 2048: max |gpu - oracle| <= 1e-2 * RMS(oracle) per matmul;
- decode logits: max |gpu - cpu| <= 1e-2 * RMS(cpu), the parity bar of
  one matmul, held by the whole step (measured 0.9-2.0e-3 at 2 and 36 layers:
  the device and the restatement round to bf16 at the same points, so only
  the f32 summation order differs, and a value rounded the other way moves by
  one bf16 ulp, 2^-8);
- the greedy token equals argmax of the device's logits, and the CPU's argmax
  wherever the CPU's top two logits are further apart than twice that bound;
- the HIP-graph replay of a step gives the eager step's logits bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle as O
from _decode_ref import decode_ref
from _util import assert_bf16_rounded_close, assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu

H, I, V = 2048, 11008, 151936


def case(msg):
    print(f"[case] {msg}", flush=True)


def synth():
    from kriya_q4 import synth as s
    return s


def check_greedy(next_tok, logits, want, bound, what):
    """next == argmax(device logits); == argmax(cpu logits) where the CPU's top two are clearly apart."""
    assert np.array_equal(next_tok, np.argmax(logits, axis=1)), what
    for b in range(want.shape[0]):
        top2 = np.sort(want[b])[-2:]
        if top2[1] - top2[0] > 2 * bound:
            assert next_tok[b] == int(np.argmax(want[b])), f"{what}: row {b}"


@pytest.fixture(scope="module")
def lm_head(kq):
    wq = synth().q4_weight(V, H, 3501)
    return wq, q4_dev(kq, wq)


@pytest.mark.parametrize("m", [1, 16])
def test_lm_head_at_vocab_size(kq, lm_head, m):
    """kr_q4_linear with N = 151936, K = 2048, f32 logits, then kr_argmax (encoder.rs:5504-5516)."""
    case(f"LM head 151936x2048 m={m}, f32 logits + argmax")
    wq, w = lm_head
    x = synth().bf16_normal((m, H), 3510 + m)
    want = O.q4_matmul(O.Q4Planar(*wq), x)
    logits = kq.q4_linear(w, dev_bf16(x), out_dtype=kq.DTYPE_F32)
    nxt = kq.argmax(logits).cpu().numpy()
    got = logits.cpu().numpy()
    err = assert_rms_close(got, want, what=f"LM head m={m}")
    print(f"LM head m={m}: max err {err / rms(want):.2e} of RMS")
    check_greedy(nxt, got, want, 1e-2 * rms(want), f"LM head m={m}")


def rmsnorm_np(h_bits, ln_bits, eps=1e-6):
    """kr_rmsnorm's result (transformer_glue.metal:158-205): bf16(x * rsqrt(mean(x^2) + eps) * w)."""
    xf, wf = O.bf16_to_f32(h_bits), O.bf16_to_f32(ln_bits)
    r = 1.0 / np.sqrt((xf.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + eps)
    return O.f32_to_bf16((xf * r * wf).astype(np.float32))


@pytest.mark.parametrize("m", [1, 9, 16])
def test_fused_norm_calls_at_hidden_2048(kq, m):
    """kr_rmsnorm_q4_qkv and kr_rmsnorm_q4_mlp at the cfg3 width (q 2048, k/v 256 with biases; MLP
    2048 x 11008) against a numpy RMSNorm followed by the oracle's matmuls.  m = 1 fuses the norm into
    the GEMVs, m = 9 and 16 into the few-token kernel's staging of x."""
    s = synth()
    case(f"fused rmsnorm + qkv / mlp at H=2048, m={m}, vs numpy norm + oracle")
    h0 = s.bf16_normal((m, H), 3520 + m, std=3.0)
    ln = O.f32_to_bf16(1.0 + O.bf16_to_f32(s.bf16_normal((H,), 3521, std=0.1)))
    x = rmsnorm_np(h0, ln)
    shapes = ((2048, H), (256, H), (256, H))
    wq = [s.q4_weight(n, k, 3522 + i) for i, (n, k) in enumerate(shapes)]
    bq = [s.bf16_normal((n,), 3530 + i, std=0.1) for i, (n, _) in enumerate(shapes)]
    got = kq.rmsnorm_qkv(dev_bf16(h0), dev_bf16(ln), 1e-6, *(q4_dev(kq, w) for w in wq),
                         *(dev_bf16(b) for b in bq), out_dtype=kq.DTYPE_F32)
    for name, g_, w_, b_ in zip("qkv", got, wq, bq):
        want = O.q4_matmul(O.Q4Planar(*w_), x) + O.bf16_to_f32(b_)
        assert_rms_close(g_.cpu().numpy(), want, what=f"fused {name} m={m}")
    gw, uw = s.q4_weight(I, H, 3540), s.q4_weight(I, H, 3541)
    dw = s.q4_weight(H, I, 3542)
    delta = O.q4_mlp(O.Q4Planar(*gw), O.Q4Planar(*uw), O.Q4Planar(*dw), x)
    hd = dev_bf16(h0).clone()
    kq.rmsnorm_mlp(q4_dev(kq, gw), q4_dev(kq, uw), q4_dev(kq, dw), hd, dev_bf16(ln), 1e-6)
    assert_bf16_rounded_close(host_bits(hd), O.bf16_to_f32(h0) + delta, rms(delta), rel=1e-2,
                              what=f"fused mlp m={m}")


def run_step(m):
    """One eager step; returns (tokens, positions, caches before the step, logits, next)."""
    tokens = m.tokens.cpu().numpy().copy()
    pos = m.positions.cpu().numpy().copy()
    caches0 = [(L.k_cache.clone(), L.v_cache.clone()) for L in m.layers]
    nxt = m.step()
    torch.cuda.synchronize()
    return tokens, pos, caches0, m.logits.cpu().numpy(), nxt.cpu().numpy()


@pytest.mark.parametrize("layers", [2, 36])
@pytest.mark.parametrize("batch", [1, 16])
def test_decode_step_config3(kq, batch, layers):
    """One greedy decode step of the Qwen2.5-3B-shaped model at context 512 against the CPU
    restatement (36 layers is config 3 itself); then the same step as a HIP-graph replay."""
    from kriya_q4.qwen_decode import QWEN25_3B, QwenQ4Decoder
    import dataclasses
    cfg = dataclasses.replace(QWEN25_3B, layers=layers)
    case(f"decode step cfg3 shape, {layers} layers, batch={batch}, ctx 512, vocab {cfg.vocab}")
    m = QwenQ4Decoder(cfg, batch=batch, ctx=512, seed=3600 + batch + layers)
    tokens, pos, caches0, logits, nxt = run_step(m)
    assert np.isfinite(logits).all()
    # the same step captured in a HIP graph and replayed from the same tokens: the same bits
    m.tokens.copy_(torch.from_numpy(tokens).cuda())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            m.step()
    torch.cuda.current_stream().wait_stream(s)
    for replay in range(2):
        m.tokens.copy_(torch.from_numpy(tokens).cuda())
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(m.logits.cpu().numpy().view(np.uint32), logits.view(np.uint32)), f"replay {replay}"
        assert np.array_equal(m.next.cpu().numpy(), nxt)
    del g
    for L, (kc, vc) in zip(m.layers, caches0):  # the restatement starts from the caches before the step
        L.k_cache, L.v_cache = kc, vc
    want = decode_ref(m, cfg, tokens, pos)
    err = assert_rms_close(logits, want, rel=1e-2, what=f"decode logits B={batch} layers={layers}")
    print(f"decode B={batch} layers={layers}: max logit err {err / rms(want):.2e} of RMS")
    check_greedy(nxt, logits, want, 1e-2 * rms(want), f"decode B={batch} layers={layers}")
    del m
    torch.cuda.empty_cache()
