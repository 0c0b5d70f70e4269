"""Local checkpoint loading (SafeTensors parse, shard discovery, the Llama
alias map) against the reference's own parse cases (engine.test.ts:415-431)
and files written by the safetensors package; then the HF fixture saved as
safetensors and loaded back through the same path the runner uses."""
import json
import os
import struct

import numpy as np
import pytest

import three_llm_amd.checkpoint as C
import three_llm_amd.weights as W


def st_bytes(tensors, metadata=None):
    """A safetensors file image: {name: (dtype, shape, raw bytes)}."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata is not None:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    return struct.pack("<II", len(hb), 0) + hb + b"".join(blobs)


def reference_fixture(dtype="F32", values=(1, 2, 3, 4)):
    """createSafeTensorsFixture, engine.test.ts:62-85."""
    raw = np.float32(values).tobytes() if dtype == "F32" else np.uint16(values).tobytes()
    return st_bytes({"values": (dtype, [2, 2], raw)})


def test_parse_reference_cases():
    _, t = C.parse_safetensors(reference_fixture())
    assert t["values"].shape == [2, 2] and t["values"].dtype == "F32"
    assert t["values"].data.tolist() == [1, 2, 3, 4]
    _, t = C.parse_safetensors(reference_fixture("F16", (0x3c00, 0x4000, 0x4200, 0x4400)))
    assert t["values"].dtype == "F16" and t["values"].data.tolist() == [0x3c00, 0x4000, 0x4200, 0x4400]
    assert t["values"].fp32().tolist() == [[1, 2], [3, 4]]
    with pytest.raises(C.SafeTensorsError, match="data extends beyond the file"):
        C.parse_safetensors(reference_fixture()[:-1])
    with pytest.raises(C.SafeTensorsError, match="too small to contain a header"):
        C.parse_safetensors(bytes(7))


def test_parse_rejects_malformed_headers():
    good = reference_fixture()
    with pytest.raises(C.SafeTensorsError, match="Header extends beyond the file"):
        C.parse_safetensors(struct.pack("<II", 1000, 0) + b"{}")
    with pytest.raises(C.SafeTensorsError, match="Header is too large"):
        C.parse_safetensors(struct.pack("<II", 2, 1) + b"{}")

    def with_header(h, data=b""):
        hb = json.dumps(h).encode()
        return struct.pack("<II", len(hb), 0) + hb + data

    with pytest.raises(C.SafeTensorsError, match="invalid descriptor"):
        C.parse_safetensors(with_header({"x": 3}))
    with pytest.raises(C.SafeTensorsError, match='Unsupported dtype "F64"'):
        C.parse_safetensors(with_header({"x": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}, bytes(8)))
    with pytest.raises(C.SafeTensorsError, match="invalid shape"):
        C.parse_safetensors(with_header({"x": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, bytes(4)))
    with pytest.raises(C.SafeTensorsError, match="invalid data offsets"):
        C.parse_safetensors(with_header({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}, bytes(4)))
    with pytest.raises(C.SafeTensorsError, match="has 8 bytes, expected 4"):
        C.parse_safetensors(with_header({"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 8]}}, bytes(8)))
    meta, t = C.parse_safetensors(st_bytes({"a": ("U8", [3], b"\x01\x02\x03")}, {"format": "pt"}))
    assert meta == {"format": "pt"} and t["a"].data.tolist() == [1, 2, 3]
    _, t = C.parse_safetensors(good, keep_tensor=lambda n: False)
    assert t == {}


def test_parse_files_written_by_safetensors_package(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(0)
    arrays = {"a": rng.standard_normal((3, 5)).astype(np.float32),
              "b": rng.standard_normal(7).astype(np.float16),
              "c": np.arange(6, dtype=np.int64).reshape(2, 3)}
    path = tmp_path / "model.safetensors"
    st.save_file(arrays, str(path))
    tensors = C.load_safetensors_model(str(tmp_path))
    assert np.array_equal(tensors["a"].fp32(), arrays["a"])
    assert np.array_equal(tensors["b"].fp32(), arrays["b"].astype(np.float32))
    assert tensors["c"].data.reshape(2, 3).tolist() == arrays["c"].tolist()


def test_bf16_widening_is_exact():
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    t = C.Tensor("x", "BF16", [len(bits)], bits)
    got = t.fp32().view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_shard_discovery(tmp_path):
    (tmp_path / "a.safetensors").write_bytes(st_bytes({"x": ("F32", [1], np.float32([1]).tobytes())}))
    (tmp_path / "b.safetensors").write_bytes(st_bytes({"y": ("F32", [1], np.float32([2]).tobytes())}))
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"y": "b.safetensors", "x": "a.safetensors", "z": "b.safetensors"}}))
    assert C.resolve_safetensor_files(str(tmp_path)) == ["b.safetensors", "a.safetensors"]
    t = C.load_safetensors_model(str(tmp_path))
    assert t["x"].data.tolist() == [1] and t["y"].data.tolist() == [2]
    (tmp_path / "model.safetensors").write_bytes(st_bytes({"w": ("F32", [1], np.float32([3]).tobytes())}))
    assert C.resolve_safetensor_files(str(tmp_path)) == ["model.safetensors"]


def test_alias_map_and_prefix():
    one = np.zeros(1, np.float32)
    for prefix in ("model.", "", "language_model.", "model.language_model."):
        ts = {prefix + "embed_tokens.weight": one, prefix + "layers.0.self_attn.q_proj.weight": one}
        assert C.detect_language_prefix(ts) == prefix
        assert C.resolve_tensor(ts, prefix, "attn_q", 0) is one
        assert C.resolve_tensor(ts, prefix, "output") is one  # tied: falls back to the embedding
    with pytest.raises(C.TensorNameError, match=r'Missing "attn_k" \(llama\). Tried: model.layers.3.self_attn.k_proj'):
        C.resolve_tensor({"model.embed_tokens.weight": one}, "model.", "attn_k", 3)
    with pytest.raises(C.TensorNameError, match="Unknown tensor"):
        C.resolve_tensor({}, "model.", "delta_qkv", 0)


def save_fixture(tmp_path, hf, dtype):
    """The HF fixture tensors as a two-shard checkpoint in fp32 or fp16 bits."""
    names = list(hf["tensors"])
    shards = {}
    for i, name in enumerate(names):
        v = np.asarray(hf["tensors"][name]["values"], np.float32).reshape(hf["tensors"][name]["shape"])
        raw = v.tobytes() if dtype == "F32" else v.astype(np.float16).view(np.uint16).tobytes()
        shards.setdefault(f"model-0000{i % 2 + 1}-of-00002.safetensors", {})[name] = (dtype, v.shape, raw)
    for fname, ts in shards.items():
        (tmp_path / fname).write_bytes(st_bytes(ts))
    wm = {n: f for f, ts in shards.items() for n in ts}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    (tmp_path / "config.json").write_text(json.dumps(hf["cases"][0]["config"]))


@pytest.mark.parametrize("dtype", ["F32", "F16"])
def test_fixture_checkpoint_round_trip(tmp_path, hf_fixture, dtype):
    save_fixture(tmp_path, hf_fixture, dtype)
    hw, cfg = C.load_checkpoint(str(tmp_path), W.Storage(linear="f16", head="f16", embed="f32", kv="f32"))
    tensors = {k: np.asarray(v["values"], np.float32).reshape(v["shape"]) for k, v in hf_fixture["tensors"].items()}
    if dtype == "F16":
        tensors = {k: v.astype(np.float16).astype(np.float32) for k, v in tensors.items()}
    ref = W.from_hf(cfg, tensors, W.Storage(linear="f16", head="f16", embed="f32", kv="f32"))
    assert hw.recipe == ref.recipe
    for kind, layer in ref.kinds():
        assert np.array_equal(hw.fp32(kind, layer), ref.fp32(kind, layer)), (kind, layer)


# ----------------------------------------------------------------- on GPU --

def bf16_bits(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.gpu
def test_fixture_checkpoint_on_gpu(tmp_path, hf_fixture):
    """The fixture saved as an fp16 two-shard checkpoint, loaded by
    DecoderHIPRunner.from_checkpoint: logits equal the fixture's fp16-storage
    logits at the reference's hardware tolerance (reference.browser.test.ts:16)."""
    import three_llm_amd.runner as R
    save_fixture(tmp_path, hf_fixture, "F16")
    storage = W.Storage(linear="f16", head="f16", embed="f32", kv="f32")
    runner = R.DecoderHIPRunner.from_checkpoint(str(tmp_path), {"maxTokens": 64}, storage=storage)
    case = hf_fixture["cases"][0]
    for i, tok in enumerate(hf_fixture["input_ids"][:6]):
        runner.computeToken(tok, i, True)
        logits = runner.readLogits()
        err = np.abs(logits - np.asarray(case["fp16_storage_logits"][i])) - (3e-5 + 2e-4 * np.abs(
            np.asarray(case["fp16_storage_logits"][i])))
        assert err.max() <= 0
    runner.close()


@pytest.mark.gpu
def test_bf16_checkpoint_packed_to_q4_on_gpu(tmp_path):
    """A bf16 checkpoint (tied head, QKV bias, 'model.' prefix) packed to q4 g32
    at load: logits against the oracle fed the same dequantised weights, after a
    prompt long enough for the batched prefill."""
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from bridge import close, oracle_model
    import three_llm_amd.runner as R
    cfg = {"model_type": "qwen2", "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
           "num_attention_heads": 4, "num_key_value_heads": 2, "vocab_size": 1024, "rope_theta": 1e6,
           "rms_norm_eps": 1e-6, "tie_word_embeddings": True, "max_position_embeddings": 512, "eos_token_id": -1}
    rng = np.random.default_rng(11)
    H, I, D = 256, 512, 64
    shapes = {"model.embed_tokens.weight": (1024, H), "model.norm.weight": (H,)}
    for l in range(2):
        p = f"model.layers.{l}."
        shapes.update({p + "self_attn.q_proj.weight": (4 * D, H), p + "self_attn.k_proj.weight": (2 * D, H),
                       p + "self_attn.v_proj.weight": (2 * D, H), p + "self_attn.q_proj.bias": (4 * D,),
                       p + "self_attn.k_proj.bias": (2 * D,), p + "self_attn.v_proj.bias": (2 * D,),
                       p + "self_attn.o_proj.weight": (H, 4 * D), p + "mlp.gate_proj.weight": (I, H),
                       p + "mlp.up_proj.weight": (I, H), p + "mlp.down_proj.weight": (H, I),
                       p + "input_layernorm.weight": (H,), p + "post_attention_layernorm.weight": (H,)})
    ts = {}
    for name, shp in shapes.items():
        v = (1 + 0.1 * rng.standard_normal(shp)) if "norm" in name else rng.standard_normal(shp) * 0.02
        ts[name] = ("BF16", shp, bf16_bits(v).tobytes())
    (tmp_path / "model.safetensors").write_bytes(st_bytes(ts))
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    runner = R.DecoderHIPRunner.from_checkpoint(str(tmp_path), {"maxTokens": 256})
    assert runner.batchedPrefill and runner.weights.host.recipe.tied_embeddings
    om = oracle_model(runner.weights.host, 256, kv_f16=True)
    prompt = [int(t) for t in rng.integers(0, 1024, 100)]
    runner.prefillTokens(prompt, 0, len(prompt) - 1)
    for i, t in enumerate(prompt[:-1]):
        om.prefill(t, i)
    runner.computeToken(prompt[-1], len(prompt) - 1, True)
    close(runner.readLogits(), om.forward(prompt[-1], len(prompt) - 1), 2e-2, 1e-2)
    runner.close()
    om.close()
    # with a tokenizer beside the weights: text in, text out (generate.ts:210-305)
    tk = pytest.importorskip("tokenizers")
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers
    hf = Tokenizer(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    hf.train_from_iterator(["Once upon a time there was a little robot named Bolt. " * 20],
                           trainers.BpeTrainer(vocab_size=400, special_tokens=["<|endoftext|>"],
                                               initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                               show_progress=False))
    hf.model.save(str(tmp_path))
    runner = R.DecoderHIPRunner.from_checkpoint(str(tmp_path), {"maxTokens": 256})
    prompt_text = "Once upon a time there was a little robot"
    ids = runner.weights.tokenizer.encode(prompt_text)
    assert ids == hf.encode(prompt_text).ids
    res = runner.generate(prompt_text, {"temperature": 0, "maxNewTokens": 12})
    assert res["tokens"][:len(ids)] == ids and res["promptTokens"] == len(ids)
    assert len(res["generatedTokens"]) == 12 and res["text"].startswith(prompt_text)
    runner.close()
