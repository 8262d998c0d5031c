"""CPU restatement of config 3's decode step for the GPU parity tests (test
infrastructure): one step of kriya_q4.qwen_decode.QwenQ4Decoder layer by layer,
with the oracle's Q4 matmuls, numpy RMSNorm / RoPE / attention in f64, and a
bf16 rounding wherever the device stores bf16.  Follows the reference's decode
pass (crates/kriya-backend-metal/src/encoder.rs:4880-5516)."""
import math

import numpy as np

import oracle as O


def bf(a):
    """round f32 values to bf16 (RNE) and back"""
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(a, np.float32)))


def planar(m):
    return O.Q4Planar(m.qw.cpu().numpy().view(np.uint32), m.scales.cpu().numpy().view(np.uint16),
                      m.biases.cpu().numpy().view(np.uint16))


def f32(t):
    return t.float().cpu().numpy()


def rope_np(x, pos, cos_sin):
    """pairs (d, d + D/2) rotated by the table row of `pos`"""
    D = x.shape[-1]
    h = D // 2
    c, s = cos_sin[pos, :, 0], cos_sin[pos, :, 1]
    x0, x1 = x[..., :h], x[..., h:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def attention_np(q, kc, vc, pos, q_heads, kv_heads):
    """q [H, D]; kc, vc [ctx, KVH, D]; positions 0..pos"""
    D = q.shape[-1]
    out = np.empty_like(q)
    for h in range(q_heads):
        kvh = h // (q_heads // kv_heads)
        k = kc[: pos + 1, kvh].astype(np.float64)
        v = vc[: pos + 1, kvh].astype(np.float64)
        sc = k @ q[h].astype(np.float64) / math.sqrt(D)
        p = np.exp(sc - sc.max())
        out[h] = (p @ v) / p.sum()
    return out


def decode_ref(m, cfg, tokens, pos):
    """CPU restatement of one decode step (qwen_decode.QwenQ4Decoder.step)."""
    B = len(tokens)
    H, KVH, D = cfg.q_heads, cfg.kv_heads, cfg.head_dim
    cs = m.cos_sin.cpu().numpy()
    E = planar(m.embed)
    h = bf(O.dequant_planar(E)[tokens])

    def rms(v, w):
        s = 1.0 / np.sqrt((v.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + cfg.eps)
        return bf(v * s * f32(w))

    def mm(W, v):
        return O.q4_matmul(W, O.f32_to_bf16(v))

    for L in m.layers:
        x = rms(h, L.ln1)
        q = bf(mm(planar(L.q), x) + f32(L.bq))
        k = bf(mm(planar(L.k), x) + f32(L.bk))
        v = bf(mm(planar(L.v), x) + f32(L.bv))
        kc = f32(L.k_cache).copy()
        vc = f32(L.v_cache).copy()
        att = np.empty_like(q)
        for b in range(B):
            qb = bf(rope_np(q[b].reshape(H, D), pos[b], cs))
            kc[b, pos[b]] = bf(rope_np(k[b].reshape(KVH, D), pos[b], cs))
            vc[b, pos[b]] = v[b].reshape(KVH, D)
            att[b] = bf(attention_np(qb, kc[b], vc[b], pos[b], H, KVH)).reshape(-1)
        h = bf(h + mm(planar(L.o), att))
        x = rms(h, L.ln2)
        g = mm(planar(L.gate), x)
        u = mm(planar(L.up), x)
        a = bf(g / (1.0 + np.exp(-g)) * u)
        h = bf(h + mm(planar(L.down), a))
    x = rms(h, m.ln_f)
    return mm(E, x)
