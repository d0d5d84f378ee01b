"""Host loaders through the C ABI (no GPU): safetensors checkpoints, the INT8
block-32 overlay and model configs, against the reference's own loader test
(tests/quantized_loader.rs) and the validation rules of src/checkpoint.rs,
src/cpu/quantized.rs:239-369 and src/model/config.rs:71-115. SHA-256 is
checked against hashlib."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import uocr_moe as um
import model_files as mf

FORMAT_ERR, JSON_ERR, SHAPE_ERR, UNSUP_ERR, NUM_ERR = um.FORMAT, um.JSON, um.SHAPE, \
    um.UNSUPPORTED, um.NUMERICAL


def status_of(fn, *args):
    try:
        fn(*args)
    except um.UocrError as e:
        return e.status
    return um.OK


# ------------------------------------------------------------ safetensors

def test_checkpoint_round_trip_and_sha256(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    b = rng.integers(-128, 127, size=(7,), dtype=np.int8)
    c = np.arange(4, dtype=np.int64)
    tensors = {"b.i8": ("I8", b.shape, b.tobytes()), "a.f32": ("F32", a.shape, a.tobytes()),
               "c.i64": ("I64", c.shape, c.tobytes()), "d.bf16": mf.bf16(a[:2])}
    path = tmp_path / "x.safetensors"
    mf.write(path, tensors, {"k": "v"})
    ck = um.Checkpoint(path)
    assert ck.names() == sorted(tensors)
    assert ck.metadata("k") == "v" and ck.metadata("missing") is None
    for name, (dtype, shape, raw) in tensors.items():
        assert ck.tensor(name) == (dtype, list(shape), raw)
    assert ck.sha256() == hashlib.sha256(path.read_bytes()).hexdigest()
    assert status_of(ck.tensor, "nope") == FORMAT_ERR


@pytest.mark.parametrize("size", [0, 1, 47, 48, 55, 56, 63, 64, 65, 119, 128, 1000, (1 << 20) + 7,
                                  (3 << 20) - 1])
def test_sha256_against_hashlib(tmp_path, size):
    # Payload sizes around the 64-byte block and the 1 MiB read boundaries.
    raw = np.random.default_rng(size).integers(0, 256, size=size, dtype=np.uint8).tobytes()
    path = tmp_path / "h.safetensors"
    mf.write(path, {"t": ("I8", [size], raw)})
    assert um.Checkpoint(path).sha256() == hashlib.sha256(path.read_bytes()).hexdigest()


def _raw(path, header: dict, payload: bytes, length=None):
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text) if length is None else length) + text + payload)


@pytest.mark.parametrize("case,expect", [
    ("short", FORMAT_ERR), ("huge_header", FORMAT_ERR), ("truncated", FORMAT_ERR),
    ("bad_json", JSON_ERR), ("bad_dtype", JSON_ERR), ("bad_shape", JSON_ERR),
    ("length_mismatch", FORMAT_ERR), ("past_end", FORMAT_ERR), ("gap", FORMAT_ERR),
    ("overlap", FORMAT_ERR), ("trailing", FORMAT_ERR), ("overflow", FORMAT_ERR),
    ("metadata_not_string", JSON_ERR),
])
def test_checkpoint_rejects(tmp_path, case, expect):
    """src/checkpoint.rs:114-178."""
    p = tmp_path / "bad.safetensors"
    t = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    payload = bytes(8)
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "huge_header":
        _raw(p, {"a": t}, payload, length=100_000_001)
    elif case == "truncated":
        _raw(p, {"a": t}, b"", length=10_000)
    elif case == "bad_json":
        p.write_bytes(struct.pack("<Q", 5) + b"{oops")
    elif case == "bad_dtype":
        _raw(p, {"a": dict(t, dtype="F64")}, payload)
    elif case == "bad_shape":
        _raw(p, {"a": dict(t, shape=[-2])}, payload)
    elif case == "length_mismatch":
        _raw(p, {"a": dict(t, shape=[3])}, payload)
    elif case == "past_end":
        _raw(p, {"a": dict(t, data_offsets=[8, 16])}, payload)
    elif case == "gap":
        _raw(p, {"a": dict(t, shape=[1], data_offsets=[4, 8])}, payload)
    elif case == "overlap":
        _raw(p, {"a": t, "b": dict(t, shape=[1], data_offsets=[4, 8])}, payload)
    elif case == "trailing":
        _raw(p, {"a": dict(t, shape=[1], data_offsets=[0, 4])}, payload)
    elif case == "overflow":
        _raw(p, {"a": dict(t, shape=[1 << 62, 8])}, payload)
    elif case == "metadata_not_string":
        _raw(p, {"__metadata__": {"x": 1}, "a": t}, payload)
    assert status_of(um.Checkpoint, p) == expect


def test_checkpoint_missing_file_is_io(tmp_path):
    assert status_of(um.Checkpoint, tmp_path / "absent.safetensors") == um.IO


# ------------------------------------------------ overlay (reference fixture)

def _fixture(d):
    """tests/quantized_loader.rs:15-33: lm_head [1, 2] = [1, -2] in F32 and its
    overlay (int8 [1, -2], scale 1.0), with the manifest."""
    source = d / "source.safetensors"
    mf.write(source, {"lm_head.weight": ("F32", [1, 2], struct.pack("<2f", 1.0, -2.0))})
    h = mf.sha256(source)
    path = d / "q.safetensors"
    data = mf.write(path, {"lm_head.weight": ("I8", [1, 2], bytes([1, 254])),
                           "lm_head.weight.q8_scales": ("F32", [1, 1], struct.pack("<f", 1.0))},
                    {"format": mf.FORMAT, "block_size": "32", "source_sha256": h})
    mf.write_manifest(path, h, data, 1)
    return source, path, h


def test_reference_overlay_fixture_validates(tmp_path):
    source, path, _ = _fixture(tmp_path)
    ck = um.Checkpoint(source)
    assert um.overlay_validate(path, ck) == 1
    ov = um.Checkpoint(path)
    assert ov.tensor("lm_head.weight") == ("I8", [1, 2], bytes([1, 254]))


def test_overlay_rejects_corruption_and_wrong_source(tmp_path):
    source, path, _ = _fixture(tmp_path)
    ck = um.Checkpoint(source)
    original = path.read_bytes()
    path.write_bytes(original[:-1] + bytes([original[-1] ^ 1]))
    assert status_of(um.overlay_validate, path, ck) == FORMAT_ERR
    path.write_bytes(original)
    wrong = tmp_path / "other.safetensors"
    mf.write(wrong, {"lm_head.weight": ("F32", [1, 2], bytes(8))})
    assert status_of(um.overlay_validate, path, um.Checkpoint(wrong)) == FORMAT_ERR
    assert um.overlay_validate(path, ck) == 1


@pytest.mark.parametrize("invalid,expect", [
    ("version", FORMAT_ERR), ("scale", NUM_ERR), ("shape", FORMAT_ERR), ("dtype", FORMAT_ERR),
    ("range", FORMAT_ERR), ("missing", FORMAT_ERR)])
def test_authenticated_but_invalid_overlay(tmp_path, invalid, expect):
    """tests/quantized_loader.rs:63-104: each variant is re-hashed into the
    manifest, so only the content check can reject it."""
    source, path, h = _fixture(tmp_path)
    meta = {"format": mf.FORMAT, "block_size": "32", "source_sha256": h}
    w = ("I8", [1, 2], bytes([1, 254]))
    s = ("F32", [1, 1], struct.pack("<f", 1.0))
    if invalid == "version":
        meta["format"] = "future"
    elif invalid == "scale":
        s = ("F32", [1, 1], struct.pack("<f", float("nan")))
    elif invalid == "shape":
        w = ("I8", [2, 1], w[2])
    elif invalid == "dtype":
        w = ("F16", [1, 1], w[2])
    elif invalid == "range":
        w = ("I8", [1, 2], bytes([128, 254]))
    tensors = {"lm_head.weight": w}
    if invalid != "missing":
        tensors["lm_head.weight.q8_scales"] = s
    data = mf.write(path, tensors, meta)
    mf.write_manifest(path, h, data, 1)
    assert status_of(um.overlay_validate, path, um.Checkpoint(source)) == expect


@pytest.mark.parametrize("field,value", [("schema_version", 2), ("block_size", 16),
                                         ("bytes", 1), ("matrix_count", 2)])
def test_overlay_manifest_mismatch(tmp_path, field, value):
    source, path, h = _fixture(tmp_path)
    mf.write_manifest(path, h, path.read_bytes(), 1, **{field: value})
    assert status_of(um.overlay_validate, path, um.Checkpoint(source)) == FORMAT_ERR


def test_overlay_manifest_malformed_is_json_or_io(tmp_path):
    source, path, _ = _fixture(tmp_path)
    (tmp_path / "q.json").write_text("{")
    assert status_of(um.overlay_validate, path, um.Checkpoint(source)) == JSON_ERR
    os.remove(tmp_path / "q.json")
    assert status_of(um.overlay_validate, path, um.Checkpoint(source)) == um.IO


def test_overlay_eligible_set_matches_the_model(tmp_path):
    mf.model_dir(tmp_path)
    src = tmp_path / "model-00001-of-000001.safetensors"
    mats = mf.overlay(src, tmp_path / "ov.safetensors")
    names = um.Checkpoint(src).names()
    assert sorted(mats) == sorted(n for n in names if mf.eligible(n))
    assert not any("mlp.gate.weight" in n for n in mats)  # routers stay BF16
    assert um.overlay_validate(tmp_path / "ov.safetensors", um.Checkpoint(src)) == len(mats)


# ------------------------------------------------------------------ config

def _config(tmp_path, **over):
    p = tmp_path / "config.json"
    c = mf.config_json(mf.MOE_TINY, **over)
    for k, v in list(c.items()):
        if v is None:
            del c[k]
    p.write_text(json.dumps(c))
    return p


def test_config_loads(tmp_path):
    c = um.config_load(_config(tmp_path))
    assert (c.hidden_size, c.moe_intermediate_size, c.n_routed_experts, c.num_experts_per_tok,
            c.first_k_dense_replace, c.norm_topk_prob) == (64, 64, 8, 2, 1, 1)
    assert c.rms_norm_eps == np.float32(1e-6)


@pytest.mark.parametrize("over,expect", [
    (dict(model_type="other"), UNSUP_ERR), (dict(use_mla=True), UNSUP_ERR),
    (dict(topk_method="noaux_tc"), UNSUP_ERR), (dict(rope_scaling={"type": "yarn"}), UNSUP_ERR),
    (dict(attention_bias=True), UNSUP_ERR), (dict(moe_layer_freq=2), UNSUP_ERR),
    (dict(num_experts_per_tok=9), SHAPE_ERR), (dict(num_attention_heads=3), SHAPE_ERR),
    (dict(num_key_value_heads=2), SHAPE_ERR), (dict(first_k_dense_replace=3), SHAPE_ERR),
    (dict(rms_norm_eps=0.0), SHAPE_ERR), (dict(routed_scaling_factor=-1.0), SHAPE_ERR),
    (dict(n_shared_experts=0), SHAPE_ERR), (dict(hidden_size=None), JSON_ERR),
    (dict(hidden_size=-4), JSON_ERR), (dict(use_mla="no"), JSON_ERR),
])
def test_config_rejects(tmp_path, over, expect):
    """src/model/config.rs:74-115."""
    assert status_of(um.config_load, _config(tmp_path, **over)) == expect


def test_config_rope_scaling_null_is_none(tmp_path):
    assert um.config_load(_config(tmp_path, rope_scaling=None)).hidden_size == 64
    p = tmp_path / "c2.json"
    c = mf.config_json(mf.MOE_TINY)
    c["rope_scaling"] = None
    p.write_text(json.dumps(c))
    assert um.config_load(p).hidden_size == 64


# ------------------------------------------------------------ model (no GPU)

def test_model_load_validates_before_needing_a_gpu(tmp_path):
    mf.model_dir(tmp_path)
    # Valid model, no GPU context: everything validates, then Unsupported.
    assert status_of(um.Model, None, tmp_path) == UNSUP_ERR
    # Dynamic activations need an overlay (src/model/mod.rs:87-92).
    assert status_of(um.Model, None, tmp_path, None, um.QUANT_DYNAMIC) == FORMAT_ERR


def test_model_load_shape_rules(tmp_path):
    """Decoder::new (src/decoder/mod.rs:32-88) on the MoE tensors."""
    (tmp_path / "a").mkdir()
    mf.model_dir(tmp_path / "a", drop=["model.layers.1.mlp.experts.3.up_proj.weight"])
    assert status_of(um.Model, None, tmp_path / "a") == FORMAT_ERR
    (tmp_path / "b").mkdir()
    mf.model_dir(tmp_path / "b", reshape=("model.layers.1.mlp.gate.weight", [64, 8]))
    assert status_of(um.Model, None, tmp_path / "b") == SHAPE_ERR
