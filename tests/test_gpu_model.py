"""Whole-model loading on the GPU: a model directory (config.json + safetensors)
and its INT8 overlay go through Model::load_with_quantization
(uocr_model_load), and each MoE decoder layer's experts() is compared with
the oracle on the weights read back from the same files. Also the reference
overlay fixture's product (tests/quantized_loader.rs:41-49: [-5])."""
import struct

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle as orc  # noqa: E402
import uocr_moe as um  # noqa: E402
import model_files as mf  # noqa: E402

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = um.Context(0, 1 << 28)
    yield c
    c.close()


@pytest.fixture(scope="module")
def model_files(tmp_path_factory):
    d = tmp_path_factory.mktemp("model")
    moe = mf.model_dir(d)
    mats = mf.overlay(d / "model-00001-of-000001.safetensors", d / "overlay.safetensors")
    return d, moe, mats


def oracle_layer(s, w, mats, layer, quant):
    o = orc.MoeWeights(hidden=s["hidden"], inter=s["inter"], n_experts=s["experts"],
                       top_k=s["top_k"], n_shared=s["shared"], normalize=True, scale=1.0,
                       router=w["router"], gate=w["gate"], up=w["up"], down=w["down"],
                       shared_gate=w["shared_gate"], shared_up=w["shared_up"],
                       shared_down=w["shared_down"])
    if quant != orc.QUANT_NONE:
        p = f"model.layers.{layer}.mlp."

        def stack(part):
            qs = [mats[f"{p}experts.{e}.{part}.weight"] for e in range(s["experts"])]
            return np.stack([q for q, _ in qs]), np.stack([sc for _, sc in qs])

        o.q = {"gate": stack("gate_proj"), "up": stack("up_proj"), "down": stack("down_proj"),
               "shared_gate": mats[f"{p}shared_experts.gate_proj.weight"],
               "shared_up": mats[f"{p}shared_experts.up_proj.weight"],
               "shared_down": mats[f"{p}shared_experts.down_proj.weight"]}
        o.quant_mode = quant
    return o


@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_model_directory_matches_oracle(ctx, model_files, quant, T):
    d, moe, mats = model_files
    s = mf.MOE_TINY
    say(f"model directory quant={quant} T={T}")
    overlay = None if quant == orc.QUANT_NONE else d / "overlay.safetensors"
    mode = um.QUANT_WEIGHTS_ONLY if quant != orc.QUANT_DYNAMIC else um.QUANT_DYNAMIC
    model = um.Model(ctx, d, overlay, mode)
    assert model.precision() == {orc.QUANT_NONE: "bf16_weights_fp32",
                                 orc.QUANT_WEIGHTS_ONLY: "int8_weights_fp32",
                                 orc.QUANT_DYNAMIC: "int8_weights_dynamic_activations"}[quant]
    assert not model.is_moe_layer(0) and model.is_moe_layer(1)
    x = np.random.default_rng(T + quant).standard_normal((T, s["hidden"]), dtype=np.float32)
    xd = torch.from_numpy(x).cuda()
    yd = torch.full_like(xd, float("nan"))
    torch.cuda.synchronize()
    model.experts(ctx, 1, xd, yd)
    y = yd.cpu().numpy()
    ref = orc.moe_experts(oracle_layer(s, moe[1], mats, 1, quant), x)
    err = np.max(np.abs(y - ref), axis=1) / np.maximum(np.max(np.abs(ref), axis=1), 1e-30)
    assert float(err.max()) <= 1e-3, err.max()
    with pytest.raises(um.UocrError) as e:
        model.experts(ctx, 0, xd, yd)  # a dense layer has no experts
    assert e.value.status == um.SHAPE
    model.close()


def test_reference_overlay_fixture_product(ctx, tmp_path):
    """The fixture's lm_head overlay times [3, 4] is [-5]."""
    source = tmp_path / "source.safetensors"
    mf.write(source, {"lm_head.weight": ("F32", [1, 2], struct.pack("<2f", 1.0, -2.0))})
    h = mf.sha256(source)
    path = tmp_path / "q.safetensors"
    data = mf.write(path, {"lm_head.weight": ("I8", [1, 2], bytes([1, 254])),
                           "lm_head.weight.q8_scales": ("F32", [1, 1], struct.pack("<f", 1.0))},
                    {"format": mf.FORMAT, "block_size": "32", "source_sha256": h})
    mf.write_manifest(path, h, data, 1)
    assert um.overlay_validate(path, um.Checkpoint(source)) == 1
    ov = um.Checkpoint(path)
    q = np.frombuffer(ov.tensor("lm_head.weight")[2], np.int8).reshape(1, 2)
    sc = np.frombuffer(ov.tensor("lm_head.weight.q8_scales")[2], np.float32).reshape(1, 1)
    qd, sd = torch.from_numpy(q.copy()).cuda(), torch.from_numpy(sc.copy()).cuda()
    xd = torch.tensor([[3.0, 4.0]], device="cuda")
    yd = torch.zeros((1, 1), device="cuda")
    um.int8_linear(ctx, qd, sd, xd, yd)
    assert yd.cpu().numpy().tolist() == [[-5.0]]


@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
def test_model_logits_match_oracle(ctx, model_files, quant):
    """Decoder::logits (src/decoder/mod.rs:367-379) of the last hidden row:
    RMSNorm with model.norm.weight, then lm_head.weight in BF16 or the
    overlay's INT8 (weight-only, or W8A8 under DynamicActivations)."""
    d, _, mats = model_files
    s = mf.MOE_TINY
    say(f"model logits quant={quant}")
    overlay = None if quant == orc.QUANT_NONE else d / "overlay.safetensors"
    mode = um.QUANT_WEIGHTS_ONLY if quant != orc.QUANT_DYNAMIC else um.QUANT_DYNAMIC
    model = um.Model(ctx, d, overlay, mode)
    ck = um.Checkpoint(d / "model-00001-of-000001.safetensors")
    dt, shape, raw = ck.tensor("model.norm.weight")
    assert dt == "BF16" and shape == [s["hidden"]]
    norm = orc.bf16_to_f32(np.frombuffer(raw, np.uint16))
    hidden = np.random.default_rng(7 + quant).standard_normal((3, s["hidden"]), dtype=np.float32)
    n = orc.rms_norm(hidden[-1:], norm, 1e-6)
    if quant == orc.QUANT_NONE:
        dt, shape, raw = ck.tensor("lm_head.weight")
        w = np.frombuffer(raw, np.uint16).reshape(shape)
        ref = orc.linear_weight_bf16(n, w)
    elif quant == orc.QUANT_WEIGHTS_ONLY:
        q, sc = mats["lm_head.weight"]
        ref = orc.int8_linear(q, sc, n)
    else:
        q, sc = mats["lm_head.weight"]
        ref = orc.int8_linear_dynamic(q, sc, n)
    hd = torch.from_numpy(hidden).cuda()
    out = torch.full((s["vocab"],), float("nan"), device="cuda")
    model.logits(ctx, hd, out)
    got = out.cpu().numpy().reshape(1, -1)
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    say(f"  normwise={err:.3e}")
    assert err <= 1e-5, err
    with pytest.raises(um.UocrError) as e:
        model.logits(ctx, hd[:0], out)  # no hidden state
    assert e.value.status == um.SHAPE
    model.close()
