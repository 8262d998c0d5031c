"""Config 3 (end-to-end decode) on the GPU: the Q4 embedding lookup bit-exact
against the oracle's dequantisation, the glue kernels against numpy
restatements of the reference's formulas, and one greedy decode step of a
small Qwen2-shaped model against a layer-by-layer CPU restatement that uses
the oracle's Q4 matmuls and rounds to bf16 where the device stores bf16.

Bars: embedding bit-exact; glue within a few bf16 ulps; decode-step logits
max |gpu - cpu| <= 3e-2 * RMS(cpu): the 1e-2 matmul bar per projection,
compounded over the 2 x 7 projections and the bf16 roundings between them
(one bf16 ulp is 2^-8 of a value), and the greedy token equal unless the
CPU's top two logits are closer than that bound.
"""
import numpy as np
import pytest
import torch

import oracle as O
from _decode_ref import attention_np, bf, decode_ref, rope_np
from _util import assert_rms_close, dev_bf16, host_bits, q4_dev, rms

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)


def test_embedding_bit_exact(kq):
    case("q4 embedding")
    from kriya_q4 import synth
    w = synth.q4_weight(300, 256, 3301)
    tokens = np.array([0, 299, 17, 17, 150, 300], np.int32)  # 300 is out of range -> zero row
    out = kq.embedding(kq.Q4Matrix.from_numpy(*w), torch.from_numpy(tokens).cuda())
    deq = O.dequant_planar(O.Q4Planar(*w))
    want = O.f32_to_bf16(deq[np.minimum(tokens, 299)])
    want[-1] = 0
    assert np.array_equal(host_bits(out), want)


def test_rmsnorm(kq):
    case("rmsnorm")
    from kriya_q4 import synth
    x = synth.bf16_normal((5, 320), 3302)
    w = synth.bf16_normal((320,), 3303)
    got = O.bf16_to_f32(host_bits(kq.rmsnorm(dev_bf16(x), dev_bf16(w), 1e-6)))
    xf, wf = O.bf16_to_f32(x), O.bf16_to_f32(w)
    scale = 1.0 / np.sqrt((xf.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    want = xf * scale * wf
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-6)


def test_rope_append_and_attention(kq):
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    B, H, KVH, D, ctx = 3, 8, 2, 64, 12
    case(f"rope + kv append + attention B={B} H={H}/{KVH} D={D} ctx={ctx}")
    q = synth.bf16_normal((B, H * D), 3310)
    k = synth.bf16_normal((B, KVH * D), 3311)
    v = synth.bf16_normal((B, KVH * D), 3312)
    kc = synth.bf16_normal((B, ctx, KVH, D), 3313)
    vc = synth.bf16_normal((B, ctx, KVH, D), 3314)
    pos = np.array([5, 11, 0], np.int32)
    cs = rope_table(ctx, D, 1e6)
    qd, kd, vd = dev_bf16(q), dev_bf16(k), dev_bf16(v)
    kcd, vcd = dev_bf16(kc).clone(), dev_bf16(vc).clone()
    posd = torch.from_numpy(pos).cuda()
    kq.rope_kv_append(qd, kd, vd, cs.cuda(), posd, H, KVH, D, kcd, vcd)
    att = kq.attention_decode(qd, kcd, vcd, posd, H, KVH, D)
    csn = cs.numpy()
    qf = O.bf16_to_f32(q).reshape(B, H, D)
    kf = O.bf16_to_f32(k).reshape(B, KVH, D)
    kc_want = O.bf16_to_f32(kc).copy()
    vc_want = O.bf16_to_f32(vc).copy()
    for b in range(B):
        q_rot = bf(rope_np(qf[b], pos[b], csn))
        assert np.all(np.abs(O.bf16_to_f32(host_bits(qd)).reshape(B, H, D)[b] - q_rot) <= np.abs(q_rot) * 2.0 ** -8 + 1e-6)
        kc_want[b, pos[b]] = bf(rope_np(kf[b], pos[b], csn))
        vc_want[b, pos[b]] = O.bf16_to_f32(v).reshape(B, KVH, D)[b]
    got_kc = O.bf16_to_f32(host_bits(kcd))
    assert np.all(np.abs(got_kc - kc_want) <= np.abs(kc_want) * 2.0 ** -8 + 1e-6)
    assert np.array_equal(host_bits(vcd), O.f32_to_bf16(vc_want))
    got = O.bf16_to_f32(host_bits(att)).reshape(B, H, D)
    for b in range(B):
        want = attention_np(O.bf16_to_f32(host_bits(qd)).reshape(B, H, D)[b], got_kc[b], vc_want[b], pos[b], H, KVH)
        assert np.all(np.abs(got[b] - want) <= np.abs(want) * 2.0 ** -7 + 1e-3 * np.abs(want).max())


@pytest.mark.parametrize("B,H,KVH,D,ctx,pos", [(3, 8, 2, 64, 12, [5, 11, 0]), (2, 16, 2, 128, 513, [512, 130]),
                                               (1, 4, 4, 32, 200, [199]), (2, 32, 2, 128, 70, [64, 70]),
                                               (2, 8, 4, 256, 40, [39, 17]), (1, 12, 4, 96, 33, [32]),
                                               (2, 6, 1, 8, 20, [3, 19])])
def test_rope_attention_matches_two_step_path(kq, B, H, KVH, D, ctx, pos):
    """Split-context attention with fused RoPE/append against kr_rope_kv_append + kr_attention_decode
    on the same inputs: identical caches, outputs within a few bf16 ulps (f32 summation order differs).
    The last case has positions >= max_ctx for one sequence (no append, unrotated q, whole cache)."""
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    case(f"rope+attention split B={B} H={H}/{KVH} D={D} ctx={ctx} pos={pos}")
    q = dev_bf16(synth.bf16_normal((B, H * D), 3320))
    k = dev_bf16(synth.bf16_normal((B, KVH * D), 3321))
    v = dev_bf16(synth.bf16_normal((B, KVH * D), 3322))
    kc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3323))
    vc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3324))
    cs = rope_table(ctx, D, 1e6).cuda()
    posd = torch.tensor(pos, dtype=torch.int32).cuda()
    q1, kc1, vc1 = q.clone(), kc0.clone(), vc0.clone()
    kq.rope_kv_append(q1, k, v, cs, posd, H, KVH, D, kc1, vc1)
    want = kq.attention_decode(q1, kc1, vc1, posd, H, KVH, D)
    kc2, vc2 = kc0.clone(), vc0.clone()
    got = kq.rope_attention_decode(q, k, v, cs, posd, H, KVH, D, kc2, vc2)
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    g, w = got.float().cpu().numpy(), want.float().cpu().numpy()
    assert np.all(np.abs(g - w) <= np.abs(w) * 2.0 ** -7 + 1e-3 * np.abs(w).max())


@pytest.mark.parametrize("B,H,KVH,D,ctx,pos", [(2, 16, 2, 128, 513, [512, 130]), (1, 4, 4, 256, 1024, [1023]),
                                               (2, 6, 1, 8, 20, [3, 19]), (1, 8, 2, 32, 40, [39]),
                                               (1, 8, 2, 128, 1100, [1099])])
def test_attention_merge_kernels_agree(kq, B, H, KVH, D, ctx, pos):
    """The barrier-free merge (<= 64 slices, D a power of two) against the general merge kernel on the
    same inputs: the same bits (they sum in the same order).  The last case has 69 slices, where
    both settings run the general kernel."""
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    case(f"attention merge kernels B={B} H={H}/{KVH} D={D} ctx={ctx} pos={pos}")
    q = dev_bf16(synth.bf16_normal((B, H * D), 3420))
    k = dev_bf16(synth.bf16_normal((B, KVH * D), 3421))
    v = dev_bf16(synth.bf16_normal((B, KVH * D), 3422))
    kc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3423))
    vc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3424))
    cs = rope_table(ctx, D, 1e6).cuda()
    posd = torch.tensor(pos, dtype=torch.int32).cuda()
    outs = []
    try:
        for mode in (1, 0):
            kq.set_option(kq.OPT_ATTN_MERGE_WAVE, mode)
            kc, vc = kc0.clone(), vc0.clone()
            outs.append(kq.rope_attention_decode(q, k, v, cs, posd, H, KVH, D, kc, vc).view(torch.int16).cpu())
    finally:
        kq.set_option(kq.OPT_ATTN_MERGE_WAVE, 1)
    assert torch.equal(outs[0], outs[1])
    qr = q.clone()
    kc1, vc1 = kc0.clone(), vc0.clone()
    kq.rope_kv_append(qr, k, v, cs, posd, H, KVH, D, kc1, vc1)
    want = kq.attention_decode(qr, kc1, vc1, posd, H, KVH, D).float().cpu().numpy()
    g = outs[0].view(torch.bfloat16).float().numpy()
    assert np.all(np.abs(g - want) <= np.abs(want) * 2.0 ** -7 + 1e-3 * np.abs(want).max())


@pytest.mark.parametrize("merge_wave", [1, 0])
@pytest.mark.parametrize("B,H,KVH,D,ctx,pos", [(2, 16, 2, 128, 513, [130, 7]), (1, 8, 2, 64, 1100, [40])])
def test_attention_workspace_garbage_in_empty_slices(kq, merge_wave, B, H, KVH, D, ctx, pos):
    """Slices past a sequence's length write only their (m, l); the merge must not read their
    partial sums.  The workspace is filled with 0xFF bytes (f32 NaN) before the call, and the result
    must equal the one from a zeroed workspace bit for bit.  ctx 1100 has 69 slices (general merge)."""
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    case(f"attention, NaN-filled workspace, merge_wave={merge_wave} B={B} ctx={ctx} pos={pos}")
    q = dev_bf16(synth.bf16_normal((B, H * D), 3430))
    k = dev_bf16(synth.bf16_normal((B, KVH * D), 3431))
    v = dev_bf16(synth.bf16_normal((B, KVH * D), 3432))
    kc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3433))
    vc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3434))
    cs = rope_table(ctx, D, 1e6).cuda()
    posd = torch.tensor(pos, dtype=torch.int32).cuda()
    outs = []
    try:
        kq.set_option(kq.OPT_ATTN_MERGE_WAVE, merge_wave)
        for fill in (0x00, 0xFF):
            ws = kq.attention_workspace(B, H, D, ctx)
            ws.fill_(fill)
            kc, vc = kc0.clone(), vc0.clone()
            out = kq.rope_attention_decode(q, k, v, cs, posd, H, KVH, D, kc, vc, workspace=ws)
            outs.append(out.view(torch.int16).cpu())
    finally:
        kq.set_option(kq.OPT_ATTN_MERGE_WAVE, 1)
    assert torch.isfinite(outs[1].view(torch.bfloat16).float()).all()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("m", [1, 3, 9, 16])
def test_rmsnorm_fused_qkv_and_mlp(kq, m):
    """qkv(rmsnorm(h)) and h += mlp(rmsnorm(h)) against kr_rmsnorm followed by the unfused calls:
    m = 1 fuses the norm into the GEMVs and m = 9, 16 into the few-token kernel's staging of x (the
    mean may differ in its f32 summation order, so a few normalised values may round to the
    neighbouring bf16); m = 3 runs the norm first."""
    from kriya_q4 import synth
    H, I, QN, KN = 256, 512, 256, 128
    case(f"rmsnorm fused into qkv / mlp m={m}")
    h0 = synth.bf16_normal((m, H), 3340)
    ln = dev_bf16(O.f32_to_bf16(1.0 + O.bf16_to_f32(synth.bf16_normal((H,), 3341, std=0.2))))
    ws = [q4_dev(kq, synth.q4_weight(n, H, 3342 + i)) for i, n in enumerate((QN, KN, KN))]
    bs = [dev_bf16(synth.bf16_normal((n,), 3350 + i, std=0.1)) for i, n in enumerate((QN, KN, KN))]
    h = dev_bf16(h0)
    x = kq.rmsnorm(h, ln, 1e-6)
    want = kq.qkv(*ws, x, *bs, out_dtype=kq.DTYPE_F32)
    got = kq.rmsnorm_qkv(h, ln, 1e-6, *ws, *bs, out_dtype=kq.DTYPE_F32)
    for g_, w_ in zip(got, want):
        assert_rms_close(g_.cpu().numpy(), w_.cpu().numpy(), rel=1e-2, what=f"fused qkv m={m}")
    G, U, D = (q4_dev(kq, synth.q4_weight(n, k, 3360 + i)) for i, (n, k) in enumerate(((I, H), (I, H), (H, I))))
    h_ref = dev_bf16(h0).clone()
    kq.mlp(G, U, D, h_ref, x=kq.rmsnorm(h_ref, ln, 1e-6))
    h_got = dev_bf16(h0).clone()
    kq.rmsnorm_mlp(G, U, D, h_got, ln, 1e-6)
    base = O.bf16_to_f32(h0)
    assert_rms_close(h_got.float().cpu().numpy() - base, h_ref.float().cpu().numpy() - base, rel=1e-2,
                     what=f"fused mlp m={m}")


def _argmax_dev(kq, x, split):
    """kq.argmax of a host array: one block per row (kr_argmax) or split over blocks (kr_argmax_ws)."""
    xd = torch.from_numpy(x).cuda()
    ws = kq.argmax_workspace(x.shape[0], x.shape[1]) if split else None
    return kq.argmax(xd, workspace=ws).cpu().numpy()


@pytest.mark.parametrize("split", [False, True])
def test_argmax_ties_and_nan(kq, split):
    case(f"argmax split={split}")
    x = np.random.default_rng(3).standard_normal((4, 1000)).astype(np.float32)
    x[1, 10] = x[1, 700] = 50.0          # tie -> lowest index
    x[2, :] = np.nan
    x[2, 999] = -1.0                      # NaN never wins
    x[3, 123] = np.inf
    got = _argmax_dev(kq, x, split)
    assert got.tolist() == [int(np.argmax(x[0])), 10, 999, 123]


def _argmax_ref(row):
    """Lowest index of the largest non-NaN value; 0 when every value is NaN."""
    valid = ~np.isnan(row)
    if not valid.any():
        return 0
    return int(np.flatnonzero(valid & (row == row[valid].max()))[0])


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("n", [151936, 1001, 8])
def test_argmax_quads_and_vocab_rows(kq, n, split):
    case(f"argmax n={n} split={split}: ties inside and across float4 quads, NaN next to the max, -inf rows")
    rng = np.random.default_rng(n)
    x = rng.standard_normal((8, n)).astype(np.float32)
    x[1, 5] = x[1, 6] = 60.0                          # tie inside one quad
    x[2, n - 1] = x[2, n // 2] = 60.0                 # tie across quads / threads
    x[3, 0:4] = [np.nan, 60.0, np.nan, 60.0]          # NaN beside the max in its quad
    x[4, :] = -np.inf
    x[5, :] = np.nan
    x[5, n - 2:] = [-np.inf, -np.inf]                 # only -inf besides NaN: the first -inf
    x[6, :] = -np.inf
    x[6, 3] = np.nan
    x[7, n - 1] = np.inf
    got = _argmax_dev(kq, x, split)
    want = [_argmax_ref(r) for r in x]
    assert got.tolist() == want


@pytest.mark.parametrize("rows,n", [(1, 151936), (16, 151936), (3, 4097), (2, 1027), (1, 2048)])
def test_argmax_split_block_edges(kq, rows, n):
    """kr_argmax_ws spreads a row over argmax_parts blocks: maxima tied across a block border,
    NaN runs covering whole blocks, the winner in the last (ragged) block; the same index as
    kr_argmax and as the reference rule (first maximum, NaN never taken)."""
    case(f"argmax split rows={rows} n={n}")
    parts = int(kq.lib().kr_argmax_workspace_bytes(rows, n)) // 8 // rows  # >= the true count
    rng = np.random.default_rng(rows * 100003 + n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    per = -(-n // max(1, parts))
    for r in range(rows):
        kind = r % 4
        if kind == 0 and per < n:      # equal maxima on both sides of a block border
            b = min(per * (1 + r % max(1, parts - 1)), n - 1)
            x[r, b - 1] = x[r, b] = 70.0
        elif kind == 1:                # NaN over the first half, the max in the last element
            x[r, : n // 2] = np.nan
            x[r, n - 1] = 80.0
        elif kind == 2:                # all -inf but one NaN and a later -inf run
            x[r, :] = -np.inf
            x[r, 0] = np.nan
        else:                          # the max repeated in every block: the first wins
            x[r, ::max(1, per // 2)] = 90.0
    want = [_argmax_ref(row) for row in x]
    got_split = _argmax_dev(kq, x, True)
    got_one = _argmax_dev(kq, x, False)
    assert got_split.tolist() == want
    assert got_one.tolist() == want
    # logits starting off a 16-byte boundary take the element path
    if n % 4 == 0:
        buf = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)])).cuda()
        view = buf[1:].view(rows, n)
        got = kq.argmax(view, workspace=kq.argmax_workspace(rows, n)).cpu().numpy()
        assert got.tolist() == want


@pytest.mark.parametrize("batch", [1, 3])
def test_decode_step_small_model(kq, batch):
    from kriya_q4.qwen_decode import QwenConfig, QwenQ4Decoder
    cfg = QwenConfig(hidden=256, inter=512, layers=2, vocab=384, q_heads=4, kv_heads=2, head_dim=64)
    case(f"decode step, small Qwen2-shaped model, batch={batch}")
    m = QwenQ4Decoder(cfg, batch=batch, ctx=6, seed=3400 + batch)
    tokens = m.tokens.cpu().numpy().copy()
    pos = m.positions.cpu().numpy().copy()
    caches0 = [(L.k_cache.clone(), L.v_cache.clone()) for L in m.layers]
    nxt = m.step()
    torch.cuda.synchronize()
    logits = m.logits.cpu().numpy()
    for L, (kc, vc) in zip(m.layers, caches0):  # the reference starts from the caches before the step
        L.k_cache, L.v_cache = kc, vc
    want = decode_ref(m, cfg, tokens, pos)
    assert_rms_close(logits, want, rel=3e-2, what=f"decode logits B={batch}")
    got_tok = nxt.cpu().numpy()
    assert np.array_equal(got_tok, np.argmax(logits, axis=1))
    bound = 3e-2 * np.sqrt((want.astype(np.float64) ** 2).mean())
    for b in range(batch):
        top2 = np.sort(want[b])[-2:]
        if top2[1] - top2[0] > 2 * bound:
            assert got_tok[b] == int(np.argmax(want[b]))


@pytest.mark.parametrize("B,H,KVH,ctx,pos", [(2, 16, 2, 513, [512, 130]), (1, 16, 2, 1100, [1099]),
                                             (2, 32, 2, 70, [64, 70]), (1, 8, 8, 16, [0]),
                                             (3, 16, 2, 600, [599, 0, 300]), (2, 2, 2, 40, [39, 45]),
                                             (1, 24, 2, 530, [529]), (1, 16, 2, 4200, [4100])])
def test_attention_64_position_slices(kq, B, H, KVH, ctx, pos):
    """head_dim 128 splits the context into slices of 64 positions (KR_OPT_ATTN_SLICE64 = 2 forces them; the
    default takes them when they give a block per compute unit; one wave per 16 positions over all dims, the
    block's waves merged into the slice's partial).  Against
    kr_rope_kv_append + kr_attention_decode and against 16-position slices: the same caches, outputs within
    a few bf16 ulps (the f32 sums run in another order).  pos >= ctx: no append, unrotated queries, the whole
    cache; pos 0: only the new position; ctx 4200: 66 slices, the general merge kernel."""
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    D = 128
    case(f"attention 64-position slices B={B} H={H}/{KVH} ctx={ctx} pos={pos}")
    q = dev_bf16(synth.bf16_normal((B, H * D), 3520))
    k = dev_bf16(synth.bf16_normal((B, KVH * D), 3521))
    v = dev_bf16(synth.bf16_normal((B, KVH * D), 3522))
    kc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3523))
    vc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3524))
    cs = rope_table(ctx, D, 1e6).cuda()
    posd = torch.tensor(pos, dtype=torch.int32).cuda()
    q1, kc1, vc1 = q.clone(), kc0.clone(), vc0.clone()
    kq.rope_kv_append(q1, k, v, cs, posd, H, KVH, D, kc1, vc1)
    want = kq.attention_decode(q1, kc1, vc1, posd, H, KVH, D).float().cpu().numpy()
    outs = {}
    try:
        for wide in (2, 0):
            kq.set_option(kq.OPT_ATTN_SLICE64, wide)
            kc, vc = kc0.clone(), vc0.clone()
            outs[wide] = kq.rope_attention_decode(q, k, v, cs, posd, H, KVH, D, kc, vc).float().cpu().numpy()
            assert torch.equal(kc1.view(torch.int16), kc.view(torch.int16)), f"k cache, slice64={wide}"
            assert torch.equal(vc1.view(torch.int16), vc.view(torch.int16)), f"v cache, slice64={wide}"
    finally:
        kq.set_option(kq.OPT_ATTN_SLICE64, 1)
    for wide, g in outs.items():
        assert np.all(np.isfinite(g)), wide
        assert np.all(np.abs(g - want) <= np.abs(want) * 2.0 ** -7 + 1e-3 * np.abs(want).max()), f"slice64={wide}"
    assert np.all(np.abs(outs[2] - outs[0]) <= np.abs(outs[0]) * 2.0 ** -7 + 1e-3 * np.abs(outs[0]).max())


@pytest.mark.parametrize("B,H,KVH,ctx,pos", [(1, 16, 2, 513, [512]), (1, 16, 2, 513, [130]), (1, 16, 2, 513, [0]),
                                             (1, 16, 2, 513, [600]), (1, 8, 8, 1024, [1000]), (1, 4, 1, 64, [63]),
                                             (2, 16, 2, 513, [512, 7]), (1, 16, 2, 1100, [1099])])
@pytest.mark.parametrize("h_dtype", ["bf16", "f32"])
def test_rope_attention_q4_out(kq, B, H, KVH, ctx, pos, h_dtype):
    """kr_rope_attention_q4_out: h += attention . o_proj^T.  One sequence with at most 16 slices of 64 positions
    merges the slices inside the projection's launch; within f32 summation order of kr_rope_attention_decode
    followed by kr_q4_linear (accumulate), which it is with KR_OPT_ATTN_MERGE_OPROJ = 0 (the same caches
    either way).  Also against the oracle's GEMV of the two-step attention.  Two sequences and ctx 1100
    (18 slices) take the two calls."""
    from kriya_q4 import synth
    from kriya_q4.qwen_decode import rope_table
    D, N = 128, 2048
    case(f"rope attention + o_proj B={B} H={H}/{KVH} ctx={ctx} pos={pos} h {h_dtype}")
    q = dev_bf16(synth.bf16_normal((B, H * D), 3620))
    k = dev_bf16(synth.bf16_normal((B, KVH * D), 3621))
    v = dev_bf16(synth.bf16_normal((B, KVH * D), 3622))
    kc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3623))
    vc0 = dev_bf16(synth.bf16_normal((B, ctx, KVH, D), 3624))
    wq = synth.q4_weight(N, H * D, 3625)
    wo = kq.Q4Matrix.from_numpy(*wq)
    cs = rope_table(ctx, D, 1e6).cuda()
    posd = torch.tensor(pos, dtype=torch.int32).cuda()
    h0 = synth.bf16_normal((B, N), 3626)
    outs, caches = {}, {}
    try:
        for fused in (1, 0):
            kq.set_option(kq.OPT_ATTN_MERGE_OPROJ, fused)
            kc, vc = kc0.clone(), vc0.clone()
            h = dev_bf16(h0).clone() if h_dtype == "bf16" else torch.from_numpy(O.bf16_to_f32(h0)).cuda()
            kq.rope_attention_q4_out(q, k, v, cs, posd, H, KVH, D, kc, vc, wo, h)
            outs[fused] = h.float().cpu().numpy().astype(np.float64)
            caches[fused] = (kc.view(torch.int16).cpu(), vc.view(torch.int16).cpu())
    finally:
        kq.set_option(kq.OPT_ATTN_MERGE_OPROJ, 1)
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    # the oracle's projection of the two-step attention (kr_rope_kv_append + kr_attention_decode)
    q1, kc1, vc1 = q.clone(), kc0.clone(), vc0.clone()
    kq.rope_kv_append(q1, k, v, cs, posd, H, KVH, D, kc1, vc1)
    att = host_bits(kq.attention_decode(q1, kc1, vc1, posd, H, KVH, D))
    delta = O.q4_matmul(O.Q4Planar(*wq), att).astype(np.float64)
    base = O.bf16_to_f32(h0).astype(np.float64)
    r = rms(delta)
    slack = (np.abs(base + delta) * 2.0 ** -8 if h_dtype == "bf16" else 0.0) + 2e-2 * r
    for fused, got in outs.items():
        assert np.all(np.abs(got - (base + delta)) <= slack), f"fused={fused}"
    assert np.all(np.abs(outs[1] - outs[0]) <= slack)
