"""The checkpoint reader (include/kriya_loader.h, csrc/safetensors.cpp) on the CPU:
safetensors headers, sharded indexes, the Q4 binding paths and the fail-closed
checks of the reference (safetensors_loader.rs:67-208, tensor.rs:266-275 and
:373-405, encoder.rs:306-418 and :452-591), on files written by the test.  No
GPU work: only the host side of the library runs here."""
import json
import os

import numpy as np
import pytest

import oracle as O
import _safetensors as st

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


@pytest.fixture(scope="module")
def ld():
    import kriya_q4
    from kriya_q4 import loader

    if not os.path.exists(kriya_q4.LIB_PATH):
        kriya_q4.build()
    return loader


def raises(ld, code, fn, *args, match=None, **kwargs):
    import kriya_q4
    with pytest.raises(kriya_q4.KrError) as ei:
        fn(*args, **kwargs)
    assert ei.value.code == code, str(ei.value)
    if match:
        assert match in str(ei.value), str(ei.value)


def test_reference_header_known_answer(ld, tmp_path):
    """safetensors_loader.rs:376-418: one BF16 [2, 4] tensor (16 bytes of bf16 0.5) and __metadata__."""
    p = tmp_path / "kat.safetensors"
    data = bytes([0x00, 0x3F] * 8)
    st.write(p, {"test_tensor": ("BF16", (2, 4), data)}, metadata={"format": "pt"})
    with ld.Archive(p) as a:
        assert a.names() == ["test_tensor"]
        i = a.info("test_tensor")
        assert (i["dtype"], i["shape"], i["byte_len"]) == ("BF16", [2, 4], 16)
        assert a.host_bytes("test_tensor").tobytes() == data


def test_mlx_repack_known_answer_through_a_file(ld, tmp_path):
    """safetensors_loader.rs:420-434 (0xAB nibbles, scales 0x3F80/0x4000, biases 0/0x3C00) written as an
    MLX triplet of 1 row x 128 columns: Path B, bytes unchanged."""
    k = KATS["mlx_repack"]
    qw = np.frombuffer(bytes(k["weight_nibbles"]), np.uint32).reshape(1, 16)
    sc = np.array(k["scales"], np.uint16).reshape(1, 2)
    bi = np.array(k["biases"], np.uint16).reshape(1, 2)
    p = tmp_path / "mlx.safetensors"
    st.write(p, st.q4_triplet("proj", qw, sc, bi))
    with ld.Archive(p) as a:
        assert a.check_q4("proj", 1, 128) == 2
        assert a.host_bytes("proj.weight").tobytes() == bytes(k["weight_nibbles"])
        assert a.host_bytes("proj.scales").view(np.uint16).tolist() == k["expect_scale"]
        assert a.host_bytes("proj.biases").view(np.uint16).tolist() == k["expect_bias"]


def test_q4_paths_a_b_and_bare_prefix(ld, tmp_path):
    from kriya_q4 import synth
    n, k = 6, 192
    qw, sc, bi = synth.q4_weight(n, k, 71)
    blocks = O.planar_to_blocks36(O.Q4Planar(qw, sc, bi))
    tensors = {"a.weight": ("Q4_G64", (n, k), blocks.tobytes())}
    tensors.update(st.q4_triplet("b", qw, sc, bi))
    trip = st.q4_triplet("c", qw, sc, bi)
    tensors["c"] = trip.pop("c.weight")  # weight under the bare prefix (encoder.rs:394-418)
    tensors.update(trip)
    p = tmp_path / "paths.safetensors"
    st.write(p, tensors)
    with ld.Archive(p) as a:
        assert a.check_q4("a", n, k) == 1
        assert a.check_q4("b", n, k) == 2
        assert a.check_q4("c", n, k) == 2
        raises(ld, ld.KR_E_FORMAT, a.check_q4, "a", n, k + 64, match="shape")
        raises(ld, ld.KR_E_FORMAT, a.check_q4, "b", n + 1, k, match="byte length")
        raises(ld, ld.KR_E_MISSING, a.check_q4, "zzz", n, k, match="missing expected weight 'zzz'")


def test_malformed_files_fail_closed(ld, tmp_path):
    good = {"t": ("F32", (2, 2), np.ones(4, np.float32).tobytes())}
    cases = [
        (dict(header_len=0), "header length 0"),
        (dict(header_len=100 * 1024 * 1024 + 1), "header length"),
        (dict(header_len=10 ** 6), "runs past the end"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]'), "header JSON"),
        (dict(raw_header='{"t": {"dtype": "F64", "shape": [2], "data_offsets": [0, 16]}}'), "unsupported"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [3, 2], "data_offsets": [0, 16]}}'), "need 24"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}}'), "exceeds the file"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [2], "data_offsets": [16, 8]}}'), "end 8 < begin 16"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}, '
                         '"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}'), "duplicate key"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}'), "non-integer"),
        (dict(raw_header='{"t": {"dtype": "F32", "shape": [2]}}'), "data_offsets"),
        (dict(raw_header='[1, 2]'), "not a JSON object"),
    ]
    for i, (kw, msg) in enumerate(cases):
        p = tmp_path / f"bad{i}.safetensors"
        st.write(p, good, **kw)
        raises(ld, ld.KR_E_FORMAT, ld.Archive, p, match=msg)
    raises(ld, ld.KR_E_IO, ld.Archive, tmp_path / "nonexistent.safetensors")


def test_q4_triplet_dtype_checks(ld, tmp_path):
    from kriya_q4 import synth
    n, k = 4, 128
    qw, sc, bi = synth.q4_weight(n, k, 72)
    f32 = {"w.weight": ("U32", qw.shape, qw.tobytes()),
           "w.scales": ("F32", sc.shape, O.bf16_to_f32(sc).tobytes()),
           "w.biases": ("BF16", bi.shape, bi.tobytes())}
    ints = dict(st.q4_triplet("w", qw, sc, bi))
    ints["w.biases"] = ("I8", (n, 4), np.zeros(n * 4, np.int8).tobytes())
    bad_weight = dict(st.q4_triplet("w", qw, sc, bi))
    bad_weight["w.weight"] = ("BF16", (n, k // 4), qw.tobytes())
    for name, t, msg in (("f32", f32, "is F32"), ("ints", ints, "expected float"), ("bw", bad_weight, "packed U32")):
        p = tmp_path / f"{name}.safetensors"
        st.write(p, t)
        with ld.Archive(p) as a:
            raises(ld, ld.KR_E_FORMAT, a.check_q4, "w", n, k, match=msg)


def test_sharded_index(ld, tmp_path):
    """ShardedCheckpointLoader::open_sharded (safetensors_loader.rs:174-196)."""
    st.write(tmp_path / "model-00001-of-00002.safetensors", {"x": ("BF16", (4,), b"\x01\x00" * 4)})
    st.write(tmp_path / "model-00002-of-00002.safetensors", {"y": ("F16", (2,), b"\x00\x3c" * 2),
                                                            "unlisted": ("U8", (1,), b"\x07")})
    wm = {"x": "model-00001-of-00002.safetensors", "y": "model-00002-of-00002.safetensors"}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {"total_size": 12},
                                                                       "weight_map": wm}))
    with ld.Archive(tmp_path) as a:
        assert a.names() == ["x", "y"]
        assert a.info("x")["shard"] == "model-00001-of-00002.safetensors"
        assert a.info("y")["shard"] == "model-00002-of-00002.safetensors"
        raises(ld, ld.KR_E_MISSING, a.info, "unlisted")
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {
        "x": "model-00001-of-00002.safetensors", "z": "model-00001-of-00002.safetensors"}}))
    raises(ld, ld.KR_E_FORMAT, ld.Archive, tmp_path, match="does not hold it")
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "../x.safetensors"}}))
    raises(ld, ld.KR_E_FORMAT, ld.Archive, tmp_path, match="plain file name")
    os.remove(tmp_path / "model.safetensors.index.json")
    raises(ld, ld.KR_E_IO, ld.Archive, tmp_path, match="model.safetensors")


def dense_checkpoint(tmp_path, cfg, drop=(), scale_dtype="BF16", bias=True, reshape=None):
    """A tiny dense GQA decoder in the Hugging Face / MLX naming, every projection an MLX triplet."""
    from kriya_q4 import synth
    h, i, L, v, qh, kvh, d = cfg
    qd, kvd = qh * d, kvh * d
    t = {}
    seed = [900]

    def q4(name, n, k):
        seed[0] += 1
        qw, sc, bi = synth.q4_weight(n, k, seed[0])
        if scale_dtype == "F16":
            sc = np.ascontiguousarray(O.bf16_to_f32(sc).astype(np.float16)).view(np.uint16)
            bi = np.ascontiguousarray(O.bf16_to_f32(bi).astype(np.float16)).view(np.uint16)
        t.update(st.q4_triplet(name, qw, sc, bi, scale_dtype))

    def vec(name, n):
        t[name] = ("BF16", (n,), synth.bf16_normal((n,), 77).tobytes())

    q4("model.embed_tokens", v, h)
    vec("model.norm.weight", h)
    for layer in range(L):
        p = f"model.layers.{layer}"
        vec(f"{p}.input_layernorm.weight", h)
        vec(f"{p}.post_attention_layernorm.weight", h)
        for name, n, k in (("self_attn.q_proj", qd, h), ("self_attn.k_proj", kvd, h), ("self_attn.v_proj", kvd, h),
                           ("self_attn.o_proj", h, qd), ("mlp.gate_proj", i, h), ("mlp.up_proj", i, h),
                           ("mlp.down_proj", h, i)):
            q4(f"{p}.{name}", n, k)
        if bias:
            vec(f"{p}.self_attn.q_proj.bias", qd)
            vec(f"{p}.self_attn.k_proj.bias", kvd)
            vec(f"{p}.self_attn.v_proj.bias", kvd)
    for name in drop:
        t.pop(name)
    if reshape:
        name, shape = reshape
        dt, _, data = t[name]
        t[name] = (dt, shape, data)
    tmp_path.mkdir(parents=True, exist_ok=True)
    st.write(tmp_path / "model.safetensors", t)
    return tmp_path


CFG = (64, 128, 2, 96, 2, 1, 32)  # hidden, inter, layers, vocab, q heads, kv heads, head dim


def test_validate_dense_checkpoint(ld, tmp_path):
    """validate_production_checkpoint (encoder.rs:452-591) on a tiny Qwen2-shaped checkpoint: accepted as
    written, and each removal or change reported by name."""
    h, i, L, v, qh, kvh, d = CFG
    kw = dict(hidden=h, intermediate=i, layers=L, vocab=v, q_heads=qh, kv_heads=kvh, head_dim=d)
    with ld.Archive(dense_checkpoint(tmp_path / "ok", CFG)) as a:
        a.validate_dense(**kw)
        raises(ld, ld.KR_E_MISSING, a.validate_dense, **dict(kw, layers=3), match="model.layers.2")
        raises(ld, ld.KR_E_MISSING, a.validate_dense, **dict(kw, tie_word_embeddings=False), match="lm_head")
        raises(ld, ld.KR_E_FORMAT, a.validate_dense, **dict(kw, intermediate=192), match="mlp.gate_proj")
        import kriya_q4
        raises(ld, kriya_q4.KR_E_INVALID, a.validate_dense, **dict(kw, kv_heads=3))
    with ld.Archive(dense_checkpoint(tmp_path / "f16", CFG, scale_dtype="F16")) as a:
        a.validate_dense(**kw)
    with ld.Archive(dense_checkpoint(tmp_path / "nobias", CFG, bias=False)) as a:
        a.validate_dense(**dict(kw, qkv_bias=False))
        raises(ld, ld.KR_E_MISSING, a.validate_dense, **kw, match="q_proj.bias")
    drop = ("model.layers.1.mlp.down_proj.scales",)
    with ld.Archive(dense_checkpoint(tmp_path / "drop", CFG, drop=drop)) as a:
        raises(ld, ld.KR_E_MISSING, a.validate_dense, **kw, match="model.layers.1.mlp.down_proj")
    bad = ("model.layers.0.post_attention_layernorm.weight", (h // 2, 2))
    with ld.Archive(dense_checkpoint(tmp_path / "shape", CFG, reshape=bad)) as a:
        raises(ld, ld.KR_E_FORMAT, a.validate_dense, **kw, match="post_attention_layernorm")


def test_large_headers_open_in_linear_time(ld, tmp_path):
    """A MoE checkpoint names ~10^5 tensors: a 100k-entry header, and a sharded index of 100k entries over two
    shards, open within a few seconds (duplicate keys are found through a hash set, not by rescanning every
    earlier key), and a duplicate placed last in a 100k-entry header is still rejected."""
    import time

    n = 100_000
    names = [f"model.layers.{i // 1000}.mlp.experts.{i % 1000}.w" for i in range(n)]
    big = {nm: ("U8", (1,), bytes([i & 0xFF])) for i, nm in enumerate(names)}
    p = tmp_path / "big.safetensors"
    st.write(p, big)
    t0 = time.perf_counter()
    with ld.Archive(p) as a:
        assert len(a.names()) == n
        assert a.host_bytes(names[-1]).tobytes() == bytes([(n - 1) & 0xFF])
    t_file = time.perf_counter() - t0
    half = n // 2
    st.write(tmp_path / "model-00001-of-00002.safetensors", {nm: big[nm] for nm in names[:half]})
    st.write(tmp_path / "model-00002-of-00002.safetensors", {nm: big[nm] for nm in names[half:]})
    wm = {nm: f"model-0000{1 + (i >= half)}-of-00002.safetensors" for i, nm in enumerate(names)}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    t0 = time.perf_counter()
    with ld.Archive(tmp_path) as a:
        assert len(a.names()) == n
        assert a.info(names[-1])["shard"] == "model-00002-of-00002.safetensors"
    t_index = time.perf_counter() - t0
    print(f"100k-entry header {t_file:.2f} s, 100k-entry index over two shards {t_index:.2f} s")
    assert t_file < 5.0 and t_index < 10.0, (t_file, t_index)
    entries = ", ".join(f'"{nm}": {{"dtype": "U8", "shape": [1], "data_offsets": [{i}, {i + 1}]}}'
                        for i, nm in enumerate(names))
    dup = f'{{{entries}, "{names[0]}": {{"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}}}'
    p2 = tmp_path / "dup.safetensors"
    st.write(p2, {}, raw_header=dup, extra_data=bytes(n))
    raises(ld, ld.KR_E_FORMAT, ld.Archive, p2, match="duplicate key")
