"""The opt-in int8 x int8 MFMA mode (UOCR_FLAG_INT8_MFMA) of
DynamicActivations layers, an extension: every expert group, whatever its
row count, computes as Int8Matrix::linear_dynamic_int8 row by row
(src/cpu/quantized.rs:155-236).

Pins:
  * the int32 block sums of every routed row (gate/up on the layer input,
    down on the GPU's own FP32 hidden row, which the oracle quantises again)
    equal the oracle's linear_dynamic_int8 sums bit for bit;
  * the outputs match the oracle run one token at a time — at one token
    every group is a single row, so the oracle applies the reference's own
    W8A8 path to all of them (src/decoder/mod.rs:103-104) — within 3e-3
    normwise (a hidden value one ulp away can move one int8 step);
  * the mode needs a DynamicActivations overlay (else Unsupported).
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle as orc  # noqa: E402
import uocr_moe as um  # noqa: E402
from uocr_moe import synthetic as syn  # noqa: E402

pytestmark = pytest.mark.gpu

FULL = dict(hidden=1280, inter=896, experts=64, shared=2)
H, I, E, SH, K = 1280, 896, 64, 2, 6
W8A8_TOL = 3e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def normwise(a, b):
    return float((np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)).max())


@pytest.fixture(scope="module")
def setup():
    ctx = um.Context(0, 1 << 30)
    w = syn.moe_weights(seed=5, norm=True, **FULL)
    q = syn.int8_overlay(seed=6, **FULL)
    cfg = um.config(H, I, E, SH, K, normalize=True)
    layer = um.MoeLayer(ctx, cfg, w, um.MEMORY_HOST)
    layer.attach_int8(ctx, q, um.MEMORY_HOST, um.QUANT_DYNAMIC)
    wo = um.MoeLayer(ctx, cfg, w, um.MEMORY_HOST)
    wo.attach_int8(ctx, q, um.MEMORY_HOST, um.QUANT_WEIGHTS_ONLY)
    ow = orc.MoeWeights(hidden=H, inter=I, n_experts=E, top_k=K, n_shared=SH, normalize=True,
                        router=w["router"], gate=w["gate"], up=w["up"], down=w["down"],
                        shared_gate=w["shared_gate"], shared_up=w["shared_up"],
                        shared_down=w["shared_down"], quant_mode=orc.QUANT_DYNAMIC, q=q)
    yield ctx, layer, wo, ow, q
    layer.close()
    wo.close()
    ctx.close()


def w8a8_rows(ow, x):
    """The oracle one token at a time: every group a single row (W8A8)."""
    return np.concatenate([orc.moe_experts(ow, x[t:t + 1]) for t in range(x.shape[0])])


@pytest.mark.parametrize("T", [2, 17, 64, 300, 512])
def test_int8_mode_block_sums_and_outputs(setup, T):
    ctx, layer, wo, ow, q = setup
    x = syn.activations(T, H, seed=1100 + T)
    z = lambda *shape, dt=torch.int32: torch.full(shape, -7, dtype=dt, device="cuda")
    q8 = {"gateup_sums": z(T * K, 2 * I, H // 32), "down_sums": z(T * K, H, I // 32),
          "hidden": z(T * K, I, dt=torch.float32)}
    tr = {"expert_offsets": torch.zeros(E + 1, dtype=torch.int32, device="cuda"),
          "perm_rows": torch.zeros(T * K, dtype=torch.int32, device="cuda"),
          "topk_ids": torch.zeros((T, K), dtype=torch.int32, device="cuda"), "w8a8": q8}
    xd = torch.from_numpy(x).cuda()
    yd = torch.full_like(xd, float("nan"))
    torch.cuda.synchronize()
    um.forward(ctx, layer, xd, yd, flags=um.FLAG_INT8_MFMA, trace=tr)
    torch.cuda.synchronize()
    y = yd.cpu().numpy()
    offs = tr["expert_offsets"].cpu().numpy()
    prow = tr["perm_rows"].cpu().numpy()
    g = {k: v.cpu().numpy() for k, v in q8.items()}
    counts = np.diff(offs)
    say(f"  int8 mode T={T}: groups up to {counts.max()} rows, {(counts > 1).sum()} multi-row")
    # Every routed row's block sums (a sample of positions at the larger T).
    rng = np.random.default_rng(T)
    positions = np.arange(T * K) if T * K <= 120 else rng.choice(T * K, 120, replace=False)
    expert_of = np.searchsorted(offs, np.arange(T * K), side="right") - 1
    for p in positions:
        e = expert_of[p]
        xr = x[prow[p]].reshape(1, -1)
        _, gs = orc.int8_linear_dynamic(q["gate"][0][e], q["gate"][1][e], xr, with_block_sums=True)
        _, us = orc.int8_linear_dynamic(q["up"][0][e], q["up"][1][e], xr, with_block_sums=True)
        assert np.array_equal(g["gateup_sums"][p, :I], gs), (p, e, "gate")
        assert np.array_equal(g["gateup_sums"][p, I:], us), (p, e, "up")
        _, ds = orc.int8_linear_dynamic(q["down"][0][e], q["down"][1][e],
                                        g["hidden"][p].reshape(1, -1), with_block_sums=True)
        assert np.array_equal(g["down_sums"][p], ds), (p, e, "down")
    if T >= 17:
        assert (counts > 1).any()
    # Outputs against the reference's W8A8 path applied to every row.
    rows = np.arange(T) if T <= 64 else np.sort(rng.choice(T, 48, replace=False))
    ref = w8a8_rows(ow, x[rows])
    assert np.all(np.isfinite(y))
    err = normwise(y[rows], ref)
    say(f"  normwise {err:.3e} over {len(rows)} rows")
    assert err <= W8A8_TOL, err
    # Without a trace the GEMMs run as their own kernel instantiation (no
    # block-sum stores): the same arithmetic, so the same bits.
    y2 = torch.full_like(xd, float("nan"))
    um.forward(ctx, layer, xd, y2, flags=um.FLAG_INT8_MFMA)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().view(np.uint32), y.view(np.uint32))


def test_int8_mode_needs_dynamic_activations(setup):
    ctx, layer, wo, ow, q = setup
    xd = torch.from_numpy(syn.activations(20, H, seed=3)).cuda()
    with pytest.raises(um.UocrError) as e:
        um.forward(ctx, wo, xd, torch.empty_like(xd), flags=um.FLAG_INT8_MFMA)
    assert e.value.status == um.UNSUPPORTED


def test_int8_mode_block_stack(setup):
    """uocr_moe_block_forward over two layers in int8 mode (RMSNorm with
    weight ones, W8A8 experts, residual) against the oracle token by
    token."""
    ctx, layer, wo, ow, q = setup
    T = 40
    x = syn.activations(T, H, seed=17)
    ref = x
    for _ in range(2):
        ref = ref + w8a8_rows(ow, orc.rms_norm(ref, np.ones(H, np.float32), 1e-6))
    xd = torch.from_numpy(x).cuda()
    yd = torch.full_like(xd, float("nan"))
    torch.cuda.synchronize()
    um.block_forward(ctx, [layer, layer], xd, yd, flags=um.FLAG_INT8_MFMA)
    err = normwise(yd.cpu().numpy(), ref)
    say(f"  2-layer int8 block: normwise {err:.3e}")
    assert err <= W8A8_TOL, err
