"""The allocation-free forward (uocr_moe_forward_static) against the
context forward (uocr_moe_forward) through the C ABI: the same bits on two
calls in a row, the second with fewer tokens (the static scratch keeps the
first call's contents), on each engine that fits the static scratch, and
Resource past its size. Also the oracle bar (1e-3 normwise)."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle as orc  # noqa: E402
import uocr_moe as um  # noqa: E402
from uocr_moe import synthetic as syn  # noqa: E402

pytestmark = pytest.mark.gpu

H, I, E, SH, K = 1280, 896, 64, 2, 6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def normwise(a, b):
    return float((np.abs(a - b).max(axis=1) / np.abs(b).max(axis=1)).max())


@pytest.fixture(scope="module")
def setup():
    ctx = um.Context(0, 64 << 20)
    w = syn.moe_weights(H, I, E, SH, seed=33)
    cfg = um.config(H, I, E, SH, K, normalize=True)
    layer = um.MoeLayer(ctx, cfg, w, um.MEMORY_HOST)
    q = syn.int8_overlay(H, I, E, SH, seed=34)
    qlayer = um.MoeLayer(ctx, cfg, w, um.MEMORY_HOST)
    qlayer.attach_int8(ctx, q, um.MEMORY_HOST, um.QUANT_DYNAMIC)
    ow = orc.MoeWeights(hidden=H, inter=I, n_experts=E, top_k=K, n_shared=SH, normalize=True,
                        router=w["router"], gate=w["gate"], up=w["up"], down=w["down"],
                        shared_gate=w["shared_gate"], shared_up=w["shared_up"],
                        shared_down=w["shared_down"])
    yield ctx, cfg, layer, qlayer, ow
    layer.close()
    qlayer.close()
    ctx.close()


def run_both(ctx, layer, x, flags=0):
    xd = torch.from_numpy(x).cuda()
    ya = torch.full_like(xd, float("nan"))
    yb = torch.full_like(xd, float("nan"))
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    um.forward(ctx, layer, xd, ya, flags=flags)
    um.forward_static(layer, xd, yb, flags=flags, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    return ya.cpu().numpy(), yb.cpu().numpy()


@pytest.mark.parametrize("sizes", [(100, 1), (40, 7), (16, 3)])
def test_static_forward_matches_context_forward(setup, sizes):
    ctx, cfg, layer, qlayer, ow = setup
    for T in sizes:
        for lay, name in ((layer, "bf16"), (qlayer, "w8a8")):
            say(f"static forward T={T} {name}")
            x = syn.activations(T, H, seed=500 + T)
            ya, yb = run_both(ctx, lay, x)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (T, name)
            if name == "bf16":
                ref = orc.moe_experts(ow, x)
                assert normwise(yb, ref) <= 1e-3


def test_static_forward_limits_and_errors(setup):
    ctx, cfg, layer, qlayer, ow = setup
    big = 1
    while um.scratch_bytes(cfg, big + 1) <= um.STATIC_SCRATCH_BYTES - um.STATIC_RESERVED_BYTES:
        big += 1
    say(f"largest static forward: {big} tokens")
    x = syn.activations(big, H, seed=77)
    ya, yb = run_both(ctx, layer, x)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
    xd = torch.zeros((big + 1, H), device="cuda")
    with pytest.raises(um.UocrError) as e:
        um.forward_static(layer, xd, torch.empty_like(xd))
    assert e.value.status == um.RESOURCE
    # A non-finite input row: Numerical in the caller's status word.
    bad = syn.activations(3, H, seed=78)
    bad[1, 5] = np.nan
    bd = torch.from_numpy(bad).cuda()
    status = torch.zeros((1,), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    um.forward_static(layer, bd, torch.empty_like(bd), status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == um.NUMERICAL
    # The next call clears it.
    um.forward_static(layer, bd[:1] * 0 + 1, torch.empty_like(bd[:1]), status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0


def test_static_forward_on_a_stream(setup):
    ctx, cfg, layer, qlayer, ow = setup
    x = syn.activations(24, H, seed=90)
    xd = torch.from_numpy(x).cuda()
    want = torch.empty_like(xd)
    torch.cuda.synchronize()
    um.forward(ctx, layer, xd, want)
    s = torch.cuda.Stream()
    got = torch.full_like(xd, float("nan"))
    torch.cuda.synchronize()
    um.forward_static(layer, xd, got, stream=s)
    s.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("T", [1, 24])
def test_static_forward_graph_replays(setup, T):
    """The allocation-free forward captured in a HIP graph (the one-token
    engine's single launch with its self-clearing synchronisation words at
    T = 1; router, dispatch and the MFMA engine at T = 24) and replayed four
    times, with eager forwards between the replays: every replay gives the
    eager forward's bits."""
    ctx, cfg, layer, qlayer, ow = setup
    x = syn.activations(T, H, seed=95 + T)
    xd = torch.from_numpy(x).cuda()
    want = torch.empty_like(xd)
    torch.cuda.synchronize()
    um.forward(ctx, layer, xd, want)
    s = torch.cuda.Stream()
    got = torch.full_like(xd, float("nan"))
    torch.cuda.synchronize()
    um.forward_static(layer, xd, got, stream=s)  # first call outside the capture
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        um.forward_static(layer, xd, got, stream=s)
    other = torch.empty_like(xd)
    for rep in range(4):
        say(f"graph replay T={T} #{rep}")
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), rep
        um.forward(ctx, layer, xd, other)
        torch.cuda.synchronize()
        assert torch.equal(other, want), rep
