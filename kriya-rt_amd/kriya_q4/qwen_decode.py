"""Config 3: end-to-end greedy decode of a Qwen2.5-3B-shaped model with random
Q4_G64 weights, every matmul on the Q4 kernels of libkriya_q4.

The layer follows the reference's decode pass (forward_and_sample_impl,
crates/kriya-backend-metal/src/encoder.rs:4880-5484) for a dense Qwen2 layer:

    x = rmsnorm(h, ln1)                              transformer_glue.metal:158-205
    q, k, v = x Wq^T + bq, x Wk^T + bk, x Wv^T + bv  encode_fused_qkv (:2539-2619); one launch with
                                                     the norm fused in at batch 1
    rope(q, k) at the position; append k, v          paged_gqa_and_deltanet.metal:115-222
    a = attention(q, K[0..pos], V[0..pos])           GQA decode (one split-context launch, rope and
                                                     append fused in)
    h += a Wo^T                                      encode_q4_linear_accumulate (:2497-2536); at batch 1
                                                     the slices' merge runs inside this launch
    x = rmsnorm(h, ln2)
    h += down(silu(gate x) * up x)                   encode_dense_mlp (:2851-2906); the norm fused into
                                                     the gate/up GEMV at batch 1

then logits = rmsnorm(h, ln_f) E^T with the tied Q4 embedding E (the LM head,
encoder.rs:5506-5516) and the next token = argmax (greedy sampler).

Weights are generated on the device (no checkpoint exists offline), or read
from a safetensors checkpoint with load_weights (kriya_q4.loader).  Generated:
qw uniform u32, scales bf16(|N(0, 0.02)| + 1e-3), biases bf16(-8 scale), norm
weights bf16(1 + 0.1 N), qkv biases bf16(0.1 N).  The KV cache of the first
`ctx` positions is filled with bf16 N(0, 1).
"""
from __future__ import annotations

import dataclasses
from typing import List

import torch

from . import (ACT_SWIGLU, DTYPE_BF16, DTYPE_F32, Q4Matrix, argmax, argmax_workspace, attention_q4_out_workspace,
               embedding, lib, q4_linear, rmsnorm, rmsnorm_mlp, rmsnorm_mlp_workspace, rmsnorm_qkv,
               rope_attention_q4_out)


@dataclasses.dataclass(frozen=True)
class QwenConfig:
    hidden: int = 2048
    inter: int = 11008
    layers: int = 36
    vocab: int = 151936
    q_heads: int = 16
    kv_heads: int = 2
    head_dim: int = 128
    rope_theta: float = 1e6
    eps: float = 1e-6

    def q4_bytes_per_step(self) -> int:
        per = lambda n, k: n * k // 2 + n * (k // 64) * 4  # noqa: E731
        h, i, kv = self.hidden, self.inter, self.kv_heads * self.head_dim
        layer = per(h, h) * 2 + per(kv, h) * 2 + per(i, h) * 2 + per(h, i)
        return self.layers * layer + per(self.vocab, h)


QWEN25_3B = QwenConfig()


def rope_table(max_ctx: int, head_dim: int, theta: float) -> torch.Tensor:
    """cos/sin f32 [max_ctx, head_dim/2, 2]: angle = pos * theta^(-2i/head_dim)
    (encoder.rs:1940-1950, f32 arithmetic as there)."""
    half = head_dim // 2
    i = torch.arange(half, dtype=torch.float32)
    inv_freq = torch.pow(torch.tensor(theta, dtype=torch.float32), -(2.0 * i) / float(head_dim))
    pos = torch.arange(max_ctx, dtype=torch.float32)[:, None]
    ang = pos * inv_freq[None, :]
    return torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).contiguous()


def _random_q4(n: int, k: int, gen: torch.Generator, device) -> Q4Matrix:
    qw = torch.randint(-(2 ** 31), 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=device, generator=gen)
    s = (torch.randn((n, k // 64), device=device, generator=gen).abs() * 0.02 + 1e-3).to(torch.bfloat16)
    b = (s.float() * -8.0).to(torch.bfloat16)  # exact
    return Q4Matrix(qw, s.view(torch.int16), b.view(torch.int16))


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).contiguous()


@dataclasses.dataclass
class Layer:
    ln1: torch.Tensor
    ln2: torch.Tensor
    q: Q4Matrix
    k: Q4Matrix
    v: Q4Matrix
    o: Q4Matrix
    gate: Q4Matrix
    up: Q4Matrix
    down: Q4Matrix
    bq: torch.Tensor
    bk: torch.Tensor
    bv: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor


class QwenQ4Decoder:
    """Device-resident weights, KV cache and activation buffers for `batch`
    sequences; `step()` enqueues one decode step (all on the current stream)."""

    def __init__(self, cfg: QwenConfig = QWEN25_3B, batch: int = 1, ctx: int = 512, seed: int = 3000,
                 device: str = "cuda"):
        lib()
        self.cfg, self.batch, self.ctx = cfg, batch, ctx
        self.max_ctx = ctx + 1
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        c = cfg
        kv = c.kv_heads * c.head_dim
        self.layers: List[Layer] = []
        for _ in range(c.layers):
            self.layers.append(Layer(
                ln1=_bf16(1.0 + 0.1 * torch.randn(c.hidden, device=device, generator=gen)),
                ln2=_bf16(1.0 + 0.1 * torch.randn(c.hidden, device=device, generator=gen)),
                q=_random_q4(c.q_heads * c.head_dim, c.hidden, gen, device),
                k=_random_q4(kv, c.hidden, gen, device),
                v=_random_q4(kv, c.hidden, gen, device),
                o=_random_q4(c.hidden, c.q_heads * c.head_dim, gen, device),
                gate=_random_q4(c.inter, c.hidden, gen, device),
                up=_random_q4(c.inter, c.hidden, gen, device),
                down=_random_q4(c.hidden, c.inter, gen, device),
                bq=_bf16(0.1 * torch.randn(c.q_heads * c.head_dim, device=device, generator=gen)),
                bk=_bf16(0.1 * torch.randn(kv, device=device, generator=gen)),
                bv=_bf16(0.1 * torch.randn(kv, device=device, generator=gen)),
                k_cache=_bf16(torch.randn((batch, self.max_ctx, c.kv_heads, c.head_dim), device=device,
                                          generator=gen)),
                v_cache=_bf16(torch.randn((batch, self.max_ctx, c.kv_heads, c.head_dim), device=device,
                                          generator=gen)),
            ))
        self.embed = _random_q4(c.vocab, c.hidden, gen, device)
        self.ln_f = _bf16(1.0 + 0.1 * torch.randn(c.hidden, device=device, generator=gen))
        self.cos_sin = rope_table(self.max_ctx, c.head_dim, c.rope_theta).to(device)
        # activations
        self.tokens = torch.randint(0, c.vocab, (batch,), dtype=torch.int32, device=device, generator=gen)
        self.positions = torch.full((batch,), ctx, dtype=torch.int32, device=device)
        self.h = torch.empty((batch, c.hidden), dtype=torch.bfloat16, device=device)
        self.x = torch.empty_like(self.h)
        self.q = torch.empty((batch, c.q_heads * c.head_dim), dtype=torch.bfloat16, device=device)
        self.k = torch.empty((batch, kv), dtype=torch.bfloat16, device=device)
        self.v = torch.empty_like(self.k)
        self.logits = torch.empty((batch, c.vocab), dtype=torch.float32, device=device)
        self.next = self.tokens  # greedy: the argmax writes the token the next step embeds
        self.argmax_ws = argmax_workspace(batch, c.vocab, device=device)
        self.ws = rmsnorm_mlp_workspace(batch, c.hidden, c.inter, device=device)
        self.attn_ws = attention_q4_out_workspace(batch, c.q_heads, c.head_dim, self.max_ctx, device=device)

    def load_weights(self, archive) -> None:
        """Replaces the random weights with a checkpoint's (a kriya_q4.loader.Archive in the Hugging Face /
        MLX naming, validated first as validate_production_checkpoint does, encoder.rs:452-591); the KV
        cache and token state are kept."""
        c = self.cfg
        kv = c.kv_heads * c.head_dim
        qd = c.q_heads * c.head_dim
        archive.validate_dense(c.hidden, c.inter, c.layers, c.vocab, c.q_heads, c.kv_heads, c.head_dim,
                               qkv_bias=True, tie_word_embeddings=True)
        self.embed = archive.load_q4("model.embed_tokens", c.vocab, c.hidden)
        self.ln_f = archive.load_bf16("model.norm.weight", c.hidden)
        for i, L in enumerate(self.layers):
            p = f"model.layers.{i}"
            L.ln1 = archive.load_bf16(f"{p}.input_layernorm.weight", c.hidden)
            L.ln2 = archive.load_bf16(f"{p}.post_attention_layernorm.weight", c.hidden)
            L.q = archive.load_q4(f"{p}.self_attn.q_proj", qd, c.hidden)
            L.k = archive.load_q4(f"{p}.self_attn.k_proj", kv, c.hidden)
            L.v = archive.load_q4(f"{p}.self_attn.v_proj", kv, c.hidden)
            L.o = archive.load_q4(f"{p}.self_attn.o_proj", c.hidden, qd)
            L.gate = archive.load_q4(f"{p}.mlp.gate_proj", c.inter, c.hidden)
            L.up = archive.load_q4(f"{p}.mlp.up_proj", c.inter, c.hidden)
            L.down = archive.load_q4(f"{p}.mlp.down_proj", c.hidden, c.inter)
            L.bq = archive.load_bf16(f"{p}.self_attn.q_proj.bias", qd)
            L.bk = archive.load_bf16(f"{p}.self_attn.k_proj.bias", kv)
            L.bv = archive.load_bf16(f"{p}.self_attn.v_proj.bias", kv)

    def step(self, stream=None) -> torch.Tensor:
        """One greedy decode step at `positions`; returns the next-token buffer."""
        c = self.cfg
        embedding(self.embed, self.tokens, out=self.h, stream=stream)
        for L in self.layers:
            rmsnorm_qkv(self.h, L.ln1, c.eps, L.q, L.k, L.v, q_bias=L.bq, k_bias=L.bk, v_bias=L.bv,
                        out_dtype=DTYPE_BF16, outs=(self.q, self.k, self.v), xnorm=self.x, stream=stream)
            rope_attention_q4_out(self.q, self.k, self.v, self.cos_sin, self.positions, c.q_heads, c.kv_heads,
                                  c.head_dim, L.k_cache, L.v_cache, L.o, self.h, workspace=self.attn_ws, stream=stream)
            rmsnorm_mlp(L.gate, L.up, L.down, self.h, L.ln2, c.eps, activation=ACT_SWIGLU, workspace=self.ws,
                        stream=stream)
        rmsnorm(self.h, self.ln_f, c.eps, out=self.x, stream=stream)
        q4_linear(self.embed, self.x, y=self.logits, out_dtype=DTYPE_F32, stream=stream)
        argmax(self.logits, out=self.next, workspace=self.argmax_ws, stream=stream)
        return self.next
