"""Writers for the on-disk formats the host loaders read, used to build test
fixtures: safetensors files (8-byte little-endian header length, JSON header,
payload), model directories (config.json + model-00001-of-000001.safetensors)
and INT8 block-32 overlays ("uocr-q8-block32-v1": a safetensors file of I8
matrices and F32 ".q8_scales" plus a JSON manifest beside it).

Formats: src/checkpoint.rs:114-178, src/cpu/quantized.rs:239-303,
tools/quantize.py:13-98 (written here from the format, not from that code).
"""
import hashlib
import json
import struct

import numpy as np

import oracle as orc
from uocr_moe import synthetic as syn

FORMAT = "uocr-q8-block32-v1"


def encode(tensors: dict, metadata: dict | None = None, align: bool = True) -> bytes:
    """tensors: name -> (dtype, shape, raw bytes); payload in sorted name order."""
    header, payload, offset = {}, [], 0
    for name in sorted(tensors):
        dtype, shape, raw = tensors[name]
        header[name] = {"dtype": dtype, "shape": list(shape),
                        "data_offsets": [offset, offset + len(raw)]}
        payload.append(raw)
        offset += len(raw)
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header, separators=(",", ":")).encode()
    if align:
        text += b" " * (-len(text) % 8)
    return struct.pack("<Q", len(text)) + text + b"".join(payload)


def write(path, tensors: dict, metadata: dict | None = None) -> bytes:
    data = encode(tensors, metadata)
    with open(path, "wb") as f:
        f.write(data)
    return data


def bf16(array) -> tuple:
    a = np.asarray(array, np.float32)
    return ("BF16", a.shape, syn.f32_to_bf16_bits(a).tobytes())


def bits(array_u16) -> tuple:
    a = np.ascontiguousarray(array_u16, np.uint16)
    return ("BF16", a.shape, a.tobytes())


def sha256(path) -> str:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


MOE_TINY = dict(hidden=64, inter=64, experts=8, shared=2, top_k=2, layers=2, dense=1,
                heads=4, vocab=32, intermediate=96)


def config_json(s: dict, **over) -> dict:
    c = {"model_type": "unlimited-ocr", "hidden_size": s["hidden"],
         "intermediate_size": s["intermediate"], "moe_intermediate_size": s["inter"],
         "num_hidden_layers": s["layers"], "num_attention_heads": s["heads"],
         "num_key_value_heads": s["heads"], "n_routed_experts": s["experts"],
         "n_shared_experts": s["shared"], "num_experts_per_tok": s["top_k"],
         "first_k_dense_replace": s["dense"], "use_mla": False, "vocab_size": s["vocab"],
         "rms_norm_eps": 1e-6, "norm_topk_prob": True, "routed_scaling_factor": 1.0}
    c.update(over)
    return c


def model_dir(directory, s: dict = MOE_TINY, seed: int = 5, drop=(), reshape=None) -> dict:
    """Writes a full decoder checkpoint with random BF16 weights; returns the
    MoE layers' weights (checkpoint layout, bf16 bits) by decoder layer."""
    H, I, E, S = s["hidden"], s["inter"], s["experts"], s["inter"] * s["shared"]
    rng = np.random.default_rng(seed)

    def normal(shape):
        return rng.standard_normal(shape, dtype=np.float32) * 0.05

    t, moe = {}, {}
    t["model.embed_tokens.weight"] = bf16(normal((s["vocab"], H)))
    t["lm_head.weight"] = bf16(normal((s["vocab"], H)))
    t["model.norm.weight"] = bf16(0.5 + np.arange(H) / H)
    for layer in range(s["layers"]):
        p = f"model.layers.{layer}"
        t[f"{p}.input_layernorm.weight"] = bf16(np.ones(H))
        t[f"{p}.post_attention_layernorm.weight"] = bf16(1.0 + 0.1 * normal(H))
        for part in ("q_proj", "k_proj", "v_proj", "o_proj"):
            t[f"{p}.self_attn.{part}.weight"] = bf16(normal((H, H)))
        if layer < s["dense"]:
            W = s["intermediate"]
            t[f"{p}.mlp.gate_proj.weight"] = bf16(normal((W, H)))
            t[f"{p}.mlp.up_proj.weight"] = bf16(normal((W, H)))
            t[f"{p}.mlp.down_proj.weight"] = bf16(normal((H, W)))
            continue
        w = syn.moe_weights(H, I, E, s["shared"], seed=seed * 100 + layer, norm=False)
        w["norm_weight"] = np.frombuffer(t[f"{p}.post_attention_layernorm.weight"][2], np.uint16)
        moe[layer] = w
        t[f"{p}.mlp.gate.weight"] = bits(w["router"])
        for e in range(E):
            for part, key in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
                t[f"{p}.mlp.experts.{e}.{part}.weight"] = bits(w[key][e])
        t[f"{p}.mlp.shared_experts.gate_proj.weight"] = bits(w["shared_gate"])
        t[f"{p}.mlp.shared_experts.up_proj.weight"] = bits(w["shared_up"])
        t[f"{p}.mlp.shared_experts.down_proj.weight"] = bits(w["shared_down"])
    for name in drop:
        del t[name]
    if reshape:
        name, shape = reshape
        dtype, _, raw = t[name]
        t[name] = (dtype, shape, raw)
    with open(f"{directory}/config.json", "w") as f:
        json.dump(config_json(s), f)
    write(f"{directory}/model-00001-of-000001.safetensors", t)
    return moe


def eligible(name: str) -> bool:
    """The overlay's matrix set (src/cpu/quantized.rs:268-303)."""
    if name == "lm_head.weight":
        return True
    parts = name.split(".")
    if len(parts) < 4 or parts[:2] != ["model", "layers"] or not parts[2].isdigit():
        return False
    rest = parts[3:]
    if rest[0] == "self_attn":
        return rest[1:] in (["q_proj", "weight"], ["k_proj", "weight"], ["v_proj", "weight"],
                            ["o_proj", "weight"])
    if rest[0] != "mlp":
        return False
    rest = rest[1:]
    if rest[:1] == ["shared_experts"]:
        rest = rest[1:]
    elif rest[:1] == ["experts"]:
        if len(rest) < 2 or not rest[1].isdigit():
            return False
        rest = rest[2:]
    return rest in (["gate_proj", "weight"], ["up_proj", "weight"], ["down_proj", "weight"])


def tensor_f32(dtype, shape, raw):
    if dtype == "BF16":
        return orc.bf16_to_f32(np.frombuffer(raw, np.uint16)).reshape(shape)
    return np.frombuffer(raw, np.float32).reshape(shape)


def overlay(source_path, out_path, source_tensors=None) -> dict:
    """Quantises every eligible matrix of a safetensors file (the oracle's
    Int8Matrix::quantize) into an overlay + manifest; returns name -> (q, s)."""
    from uocr_moe import Checkpoint
    ck = Checkpoint(source_path)
    t, mats = {}, {}
    for name in ck.names():
        if not eligible(name):
            continue
        dtype, shape, raw = ck.tensor(name)
        q, s = orc.int8_quantize(tensor_f32(dtype, shape, raw))
        mats[name] = (q, s)
        t[name] = ("I8", q.shape, q.tobytes())
        t[name + ".q8_scales"] = ("F32", s.shape, s.astype("<f4").tobytes())
    ck.close()
    src_hash = sha256(source_path)
    data = write(out_path, t, {"format": FORMAT, "block_size": "32", "source_sha256": src_hash})
    write_manifest(out_path, src_hash, data, len(mats))
    return mats


def write_manifest(out_path, src_hash, data: bytes, count: int, **over):
    m = {"schema_version": 1, "format": FORMAT, "block_size": 32, "source_sha256": src_hash,
         "output_sha256": hashlib.sha256(data).hexdigest(), "matrix_count": count,
         "bytes": len(data)}
    m.update(over)
    with open(str(out_path).rsplit(".", 1)[0] + ".json", "w") as f:
        json.dump(m, f)
