"""GPU parity: the HIP library (through the C ABI) against the CPU oracle on
the same seeded inputs.

Bars: top-k ids and the dispatch permutation identical except where the
oracle's logits tie within 1e-6; int8 x int8 block accumulators bit-exact;
outputs within a normwise 1e-3 (max over rows of ||y - ref||_inf /
||ref||_inf) on FP32-accumulate paths.
"""
import itertools
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle as orc  # noqa: E402
import routing_check as rc  # noqa: E402
import uocr_moe as um  # noqa: E402
from uocr_moe import synthetic as syn  # noqa: E402

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-3
TIE = 1e-6
FULL = dict(hidden=1280, inter=896, experts=64, shared=2)
SMALL = dict(hidden=128, inter=64, experts=16, shared=2)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = um.Context(0, 2 << 30)
    yield c
    c.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


_CASE_IDS = itertools.count()


class Case:
    """A layer in oracle form and uploaded to the GPU."""

    def __init__(self, ctx, shape, top_k, seed, quant=orc.QUANT_NONE, normalize=True, scale=1.0,
                 router_scale=None):
        # A serial number, not id(): a freed case's id can come back for the
        # next one, and the oracle cache must never serve one case's result
        # for another.
        self.uid = next(_CASE_IDS)
        self.shape = shape
        self.top_k = top_k
        w = syn.moe_weights(seed=seed, router_scale=router_scale, norm=True, **shape)
        self.w = w
        self.orc = orc.MoeWeights(
            hidden=shape["hidden"], inter=shape["inter"], n_experts=shape["experts"],
            top_k=top_k, n_shared=shape["shared"], normalize=normalize, scale=scale,
            router=w["router"], gate=w["gate"], up=w["up"], down=w["down"],
            shared_gate=w["shared_gate"], shared_up=w["shared_up"],
            shared_down=w["shared_down"])
        cfg = um.config(shape["hidden"], shape["inter"], shape["experts"], shape["shared"], top_k,
                        normalize=normalize, scale=scale)
        self.layer = um.MoeLayer(ctx, cfg, w, um.MEMORY_HOST)
        if quant != orc.QUANT_NONE:
            q = syn.int8_overlay(seed=seed + 1, **shape)
            self.orc.quant_mode = quant
            self.orc.q = q
            self.layer.attach_int8(ctx, q, um.MEMORY_HOST, quant)

    def run(self, ctx, x, flags=0):
        T = x.shape[0]
        E, K = self.shape["experts"], self.top_k
        tr = {"logits": torch.zeros((T, E), device="cuda"),
              "topk_ids": torch.zeros((T, K), dtype=torch.int32, device="cuda"),
              "topk_weights": torch.zeros((T, K), device="cuda"),
              "expert_offsets": torch.zeros(E + 1, dtype=torch.int32, device="cuda"),
              "perm_rows": torch.zeros(T * K, dtype=torch.int32, device="cuda"),
              "perm_weights": torch.zeros(T * K, device="cuda")}
        xd = dev(x)
        yd = torch.full_like(xd, float("nan"))
        torch.cuda.synchronize()
        um.forward(ctx, self.layer, xd, yd, flags=flags, trace=tr)
        torch.cuda.synchronize()
        return yd.cpu().numpy(), {k: v.cpu().numpy() for k, v in tr.items()}


def tie_tokens(ref_tr, gpu_tr, K):
    """Tokens whose selected set differs; raises unless each is a tie within
    1e-6 of the oracle's k-th logit."""
    return rc.tie_tokens(ref_tr.topk_ids, ref_tr.logits, gpu_tr["topk_ids"], K, tie=TIE)


def normwise(a, b):
    num = np.abs(a - b).max(axis=1)
    den = np.maximum(np.abs(b).max(axis=1), 1e-30)
    return float((num / den).max())


_REF_CACHE = {}


def oracle_ref(case, x):
    key = (case.uid, x.shape, x.tobytes())
    if key not in _REF_CACHE:
        _REF_CACHE[key] = orc.moe_experts(case.orc, x, trace=True)
    return _REF_CACHE[key]


def check_layer(case, ctx, x, tol=FP32_TOL, flags=0):
    y, tr = case.run(ctx, x, flags)
    ref, rtr = oracle_ref(case, x)
    K = case.top_k
    ties = tie_tokens(rtr, tr, K)
    keep = np.setdiff1d(np.arange(x.shape[0]), ties)
    # Routing weights of agreeing tokens: same probabilities up to exp/sum rounding.
    np.testing.assert_allclose(tr["topk_weights"][keep], rtr.topk_weights[keep], rtol=2e-5,
                               atol=1e-7)
    assert np.array_equal(tr["topk_ids"][keep], rtr.topk_ids[keep])
    # The dispatch is checked whatever the ties: exactly the stable order of
    # the GPU's own ids, and the oracle's on every token outside the ties.
    rc.check_dispatch(tr, rtr, ties, case.shape["experts"])
    assert np.all(np.isfinite(y))
    err = normwise(y[keep], ref[keep])
    say(f"  T={x.shape[0]} ties={len(ties)} normwise={err:.3e}")
    assert err <= tol, err
    return y


# ---------------------------------------------------------------- operators

def test_route_kat(ctx):
    say("route KAT (tests/moe.rs:4-13)")
    logits = dev(np.zeros((1, 4), np.float32))
    ids = torch.zeros((1, 2), dtype=torch.int32, device="cuda")
    w = torch.zeros((1, 2), device="cuda")
    um.route(ctx, logits, 2, False, 1.0, ids, w)
    assert ids.cpu().tolist() == [[0, 1]] and w.cpu().tolist() == [[0.25, 0.25]]
    um.route(ctx, logits, 2, True, 2.0, ids, w)
    assert ids.cpu().tolist() == [[0, 1]] and w.cpu().tolist() == [[1.0, 1.0]]
    with pytest.raises(um.UocrError) as e:
        um.route(ctx, dev(np.array([[0.0, np.nan]], np.float32)), 1, False, 1.0, ids, w)
    assert e.value.status == um.NUMERICAL
    with pytest.raises(um.UocrError) as e:
        um.route(ctx, dev(np.zeros((1, 1), np.float32)), 2, False, 1.0, ids, w)
    assert e.value.status == um.SHAPE


def test_route_softmax_edge_kats(ctx):
    """ops::softmax through uocr_route (tests/ops.rs:33-40, 101-132): the
    stable KAT [1000, 1000, -1000] -> [0.5, 0.5, 0] exactly; NaN, +inf and
    all -inf rows rejected; masked rows of widths 1..64 within 2e-6 of a
    float64 softmax."""
    say("softmax edge KATs on the device")
    ids = torch.zeros((1, 3), dtype=torch.int32, device="cuda")
    w = torch.zeros((1, 3), device="cuda")
    um.route(ctx, dev(np.array([[1000.0, 1000.0, -1000.0]], np.float32)), 3, False, 1.0, ids, w)
    assert ids.cpu().tolist() == [[0, 1, 2]]
    assert w.cpu().tolist() == [[0.5, 0.5, 0.0]]
    for bad in ([np.nan, 0.0], [np.inf, 0.0], [-np.inf, -np.inf], [np.inf], [-np.inf]):
        with pytest.raises(um.UocrError) as e:
            um.route(ctx, dev(np.array([bad], np.float32)), 1, False, 1.0,
                     torch.zeros((1, 1), dtype=torch.int32, device="cuda"),
                     torch.zeros((1, 1), device="cuda"))
        assert e.value.status == um.NUMERICAL, bad
    # The context recovers after the errors.
    um.route(ctx, dev(np.zeros((1, 4), np.float32)), 2, False, 1.0, ids[:, :2], w[:, :2])
    for n in [1, 3, 17, 64]:
        row = np.array([-np.inf if i % 7 == 3 else 1000 + np.sin(i * 0.37) * 30
                        for i in range(n)], np.float32)
        mx = np.float64(row.max())
        ex = np.exp(row.astype(np.float64) - mx)
        p = ex / ex.sum()
        gi = torch.zeros((1, n), dtype=torch.int32, device="cuda")
        gw = torch.zeros((1, n), device="cuda")
        um.route(ctx, dev(row.reshape(1, n)), n, False, 1.0, gi, gw)
        gi, gw = gi.cpu().numpy()[0], gw.cpu().numpy()[0]
        assert sorted(gi.tolist()) == list(range(n))
        assert np.all(np.abs(gw.astype(np.float64) - p[gi]) < 2e-6), n


def test_route_matches_oracle_on_random_rows(ctx):
    say("route vs oracle, 512 rows of 64 logits")
    rng = np.random.default_rng(1)
    lg = (rng.standard_normal((512, 64)) * 0.7).astype(np.float32)
    lg[7, :] = 0.0  # all tied: ids 0..5
    ids = torch.zeros((512, 6), dtype=torch.int32, device="cuda")
    w = torch.zeros((512, 6), device="cuda")
    um.route(ctx, dev(lg), 6, True, 1.0, ids, w)
    gi, gw = ids.cpu().numpy(), w.cpu().numpy()
    for t in range(512):
        ri, rw = orc.route_arrays(lg[t], 6, True, 1.0)
        assert np.array_equal(gi[t], ri), t
        np.testing.assert_allclose(gw[t], rw, rtol=2e-6)


def test_linear_kats(ctx):
    say("linear KAT (tests/ops.rs:10-20 without bias) and BF16 tails (tests/weights.rs:9-50)")
    x = dev(np.array([[1, 2, 3], [-1, 0, 2]], np.float32))
    wb = dev(orc.f32_to_bf16(np.array([[1, 0, -1], [2, 1, 0]], np.float32)).view(np.int16))
    y = torch.zeros((2, 2), device="cuda")
    um.linear_bf16(ctx, x, wb, y)
    assert y.cpu().numpy().ravel().tolist() == [-2.0, 4.0, -3.0, -2.0]
    for rows, cols in [(37, 131), (1025, 131), (96, 1280), (7, 64)]:
        w = np.array([((i % 29) - 14) / 16 for i in range(rows * cols)], np.float32)
        w = w.reshape(rows, cols)
        for batch in [1, 3, 20]:
            xs = np.array([((i % 13) - 6) / 8 for i in range(batch * cols)], np.float32)
            xs = xs.reshape(batch, cols)
            want = orc.linear(xs, w)
            yd = torch.zeros((batch, rows), device="cuda")
            um.linear_bf16(ctx, dev(xs), dev(orc.f32_to_bf16(w).view(np.int16)), yd)
            assert np.all(np.abs(yd.cpu().numpy() - want) < 1e-5), (rows, cols, batch)


def test_int8_linear_matches_f64(ctx):
    say("INT8 weight-only linear (tests/quantized.rs:31-73)")
    for cols in [1, 31, 32, 33, 131, 513, 64, 1280]:
        rows = 257 if cols == 513 else 7
        vals = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.37)) * 3
        vals = vals.astype(np.float32).reshape(rows, cols)
        vals[0] = 0
        q, s = orc.int8_quantize(vals)
        restored = orc.int8_dequantize(q, s)
        for batch in [1, 3]:
            x = np.cos(np.arange(batch * cols, dtype=np.float32) * np.float32(0.13))
            x = x.astype(np.float32).reshape(batch, cols)
            want = x.astype(np.float64) @ restored.astype(np.float64).T
            yd = torch.zeros((batch, rows), device="cuda")
            um.int8_linear(ctx, dev(q), dev(s), dev(x), yd)
            assert np.all(np.abs(yd.cpu().numpy() - want) < 2e-5), (cols, batch)


def test_dynamic_int8_block_sums_bit_exact(ctx):
    say("W8A8 block sums bit-exact, outputs (tests/quantized.rs:89-120)")
    for cols in [1, 15, 31, 32, 33, 131, 1280, 64, 896, 1792]:
        rows = 129 if cols >= 64 else 9
        m = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.41))
        q, s = orc.int8_quantize(m.astype(np.float32).reshape(rows, cols))
        x = (np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.17)) * 2).astype(np.float32)
        ry, rsums = orc.int8_linear_dynamic(q, s, x.reshape(1, cols), with_block_sums=True)
        yd = torch.zeros((1, rows), device="cuda")
        sums = torch.zeros(rsums.shape, dtype=torch.int32, device="cuda")
        um.int8_linear_dynamic(ctx, dev(q), dev(s), dev(x.reshape(1, cols)), yd, sums)
        assert np.array_equal(sums.cpu().numpy(), rsums), cols
        assert np.all(np.abs(yd.cpu().numpy() - ry) < 2e-4), cols
    with pytest.raises(um.UocrError) as e:
        bad = np.zeros((1, 64), np.float32)
        bad[0, 5] = np.inf
        um.int8_linear_dynamic(ctx, dev(np.zeros((2, 64), np.int8)),
                               dev(np.ones((2, 2), np.float32)), dev(bad),
                               torch.zeros((1, 2), device="cuda"))
    assert e.value.status == um.NUMERICAL


def test_rms_norm_kat(ctx):
    say("RMSNorm KAT (tests/ops.rs:42-51)")
    out = torch.zeros((1, 2), device="cuda")
    um.rms_norm(ctx, dev(np.array([[1.0, 3.0]], np.float32)), dev(np.ones(2, np.float32)), 1e-6,
                out)
    o = out.cpu().numpy().ravel()
    assert abs(o[0] - 0.44721355) < 1e-6 and abs(o[1] - 1.3416406) < 1e-6
    x = syn.activations(5, 1280, seed=3)
    w = np.linspace(0.5, 1.5, 1280).astype(np.float32)
    out = torch.zeros((5, 1280), device="cuda")
    um.rms_norm(ctx, dev(x), dev(w), 1e-6, out)
    assert normwise(out.cpu().numpy(), orc.rms_norm(x, w, 1e-6)) < 1e-6


# -------------------------------------------------------------- MoE layer

@pytest.mark.parametrize("T", [1, 2, 7, 16, 33, 100])
@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
def test_small_layer(ctx, T, quant):
    say(f"small layer T={T} quant={quant}")
    case = Case(ctx, SMALL, 4, seed=20 + T, quant=quant, normalize=(T % 2 == 0), scale=1.25)
    check_layer(case, ctx, syn.activations(T, SMALL["hidden"], seed=T))


# Expert widths beyond 1024 hold each down row of the small-batch engine as
# two column halves (single-row W8A8 groups too).
WIDE = dict(hidden=256, inter=1088, experts=8, shared=1)


@pytest.mark.parametrize("T", [1, 3, 16])
@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
def test_wide_experts_small_batch(ctx, T, quant):
    say(f"wide experts T={T} quant={quant}")
    case = Case(ctx, WIDE, 2, seed=60 + T, quant=quant)
    check_layer(case, ctx, syn.activations(T, WIDE["hidden"], seed=70 + T),
                flags=um.FLAG_FORCE_GEMV)


# Expert widths beyond 2048 exceed the small-batch engine: small batches
# take the grouped GEMM instead (and forcing the small-batch engine fails).
WIDER = dict(hidden=256, inter=2112, experts=4, shared=1)


@pytest.mark.parametrize("T", [1, 5])
@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY])
def test_widths_beyond_small_batch(ctx, T, quant):
    say(f"wider experts T={T} quant={quant}")
    case = Case(ctx, WIDER, 2, seed=80 + T, quant=quant)
    x = syn.activations(T, WIDER["hidden"], seed=90 + T)
    check_layer(case, ctx, x)
    with pytest.raises(um.UocrError) as e:
        case.run(ctx, x, flags=um.FLAG_FORCE_GEMV)
    assert e.value.status == um.UNSUPPORTED


@pytest.fixture(scope="module")
def full_bf16(ctx):
    return Case(ctx, FULL, 6, seed=0)


@pytest.fixture(scope="module")
def full_int8(ctx):
    return Case(ctx, FULL, 6, seed=0, quant=orc.QUANT_WEIGHTS_ONLY)


@pytest.fixture(scope="module")
def full_dynamic(ctx):
    return Case(ctx, FULL, 6, seed=0, quant=orc.QUANT_DYNAMIC)


@pytest.mark.parametrize("T", [1, 4, 64])
def test_full_bf16(ctx, full_bf16, T):
    say(f"full BF16 layer T={T}")
    check_layer(full_bf16, ctx, syn.activations(T, 1280, seed=100 + T))


@pytest.mark.parametrize("T", [1, 16])
def test_full_int8_weights_only(ctx, full_int8, T):
    say(f"full INT8 weight-only layer T={T}")
    check_layer(full_int8, ctx, syn.activations(T, 1280, seed=200 + T))


@pytest.mark.parametrize("T", [1, 8])
def test_full_dynamic(ctx, full_dynamic, T):
    say(f"full W8A8 layer T={T}")
    check_layer(full_dynamic, ctx, syn.activations(T, 1280, seed=300 + T))


@pytest.fixture(scope="module")
def raw_bf16(ctx):
    # The shipped model's routing mode: norm_topk_prob = false
    # (src/model/config.rs:52, tests/config.rs:9), routed_scaling_factor 1.
    return Case(ctx, FULL, 6, seed=61, normalize=False, scale=1.0)


@pytest.fixture(scope="module")
def raw_int8(ctx):
    return Case(ctx, FULL, 6, seed=62, quant=orc.QUANT_WEIGHTS_ONLY, normalize=False, scale=1.0)


@pytest.fixture(scope="module")
def raw_dynamic(ctx):
    return Case(ctx, FULL, 6, seed=63, quant=orc.QUANT_DYNAMIC, normalize=False, scale=1.0)


@pytest.mark.parametrize("kind,T,flags", [
    ("bf16", 1, 0), ("bf16", 8, 0), ("bf16", 64, 0), ("bf16", 1024, 0),
    ("bf16", 64, um.FLAG_BF16_ACTIVATIONS), ("bf16", 8, um.FLAG_FORCE_MFMA),
    ("int8", 1, 0), ("int8", 16, 0), ("int8", 512, 0),
    ("w8a8", 1, 0), ("w8a8", 12, 0), ("w8a8", 200, 0)],
    ids=lambda v: str(v))
def test_full_shape_unnormalised_routing(ctx, raw_bf16, raw_int8, raw_dynamic, kind, T, flags):
    """The unnormalised branch of moe::route (src/decoder/moe.rs:20-28:
    weights are the softmax probabilities times the scale, not renormalised
    over the chosen k) at the model shape on every engine: one-token, small
    batch, MFMA (FP32 class and BF16 activations), INT8 weight-only and
    W8A8 with single-row groups beside the MFMA GEMMs."""
    case = {"bf16": raw_bf16, "int8": raw_int8, "w8a8": raw_dynamic}[kind]
    tol = BF16_TOL if flags & um.FLAG_BF16_ACTIVATIONS else FP32_TOL
    say(f"normalize=False {kind} T={T} flags={flags}")
    check_layer(case, ctx, syn.activations(T, 1280, seed=1400 + T), tol=tol, flags=flags)


@pytest.mark.parametrize("kind", ["bf16", "int8", "w8a8"])
def test_decode_many_tokens(ctx, full_bf16, full_int8, full_dynamic, kind):
    """32 consecutive one-token forwards of different tokens at the model
    shape, each against the oracle: state carried from one decode forward
    to the next (scratch, routing, hidden values) would show here."""
    case = {"bf16": full_bf16, "int8": full_int8, "w8a8": full_dynamic}[kind]
    worst = 0.0
    for i in range(32):
        x = syn.activations(1, 1280, seed=5000 + i)
        y, _ = case.run(ctx, x)
        ref, _ = oracle_ref(case, x)
        assert np.all(np.isfinite(y)), i
        err = normwise(y, ref)
        worst = max(worst, err)
        assert err <= FP32_TOL, (i, err)
    say(f"  {kind}: 32 one-token forwards, worst normwise {worst:.3e}")


# The one-token engine at its other limits: the widest hidden row (its
# 2048-wide instantiation), 8 experts per token (10-wave down workgroups),
# an expert count that is not a multiple of 8 (a partial logit workgroup).
DECODE_EDGE = dict(hidden=2048, inter=512, experts=37, shared=2)


@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
def test_decode_edge_shapes(ctx, quant):
    case = Case(ctx, DECODE_EDGE, 8, seed=1200 + quant, quant=quant)
    for i in range(4):
        say(f"decode edge shape quant={quant} token {i}")
        check_layer(case, ctx, syn.activations(1, DECODE_EDGE["hidden"], seed=1300 + i))


@pytest.mark.parametrize("T,flags", [(5, 0), (16, 0), (40, um.FLAG_FORCE_GEMV)])
@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC])
def test_small_batch_wide_hidden(ctx, quant, T, flags):
    """The small-batch engine at a hidden width beyond 1280 (rows held in
    its 2048-wide instantiations): in INT8 weight-only layers the shared
    expert's MFMA units then head the gate/up and down launches instead of
    running beside the router; T = 40 forces the engine past 16 tokens
    (several 16-token shared tiles, the chunked dispatch)."""
    case = Case(ctx, DECODE_EDGE, 8, seed=1600 + T, quant=quant)
    say(f"small batch hidden 2048 quant={quant} T={T}")
    check_layer(case, ctx, syn.activations(T, DECODE_EDGE["hidden"], seed=1700 + T), flags=flags)


@pytest.mark.parametrize("shape,K,T,flags", [(DECODE_EDGE, 8, 17, 0),
                                             (WIDE, 2, 5, um.FLAG_FORCE_MFMA)],
                         ids=["hidden2048", "inter1088"])
def test_w8a8_singles_beside_mfma_wide(ctx, shape, K, T, flags):
    """The single-row W8A8 groups beside the MFMA engine
    (src/decoder/mod.rs:103-104) at the widths that take the other forms of
    that pass: a hidden width beyond 1280 (gate/up rows of up to 2048) and
    an expert width beyond 1024 (down rows as two column halves). The seeds
    leave 2 and 1 groups of one row."""
    case = Case(ctx, shape, K, seed=1400 + T, quant=orc.QUANT_DYNAMIC)
    x = syn.activations(T, shape["hidden"], seed=1500 + T)
    say(f"W8A8 singles beside the MFMA engine, {shape}, T={T}")
    check_layer(case, ctx, x, flags=flags)
    _, tr = case.run(ctx, x, flags)
    assert (np.diff(tr["expert_offsets"]) == 1).any()


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_decode_back_to_back(ctx, full_bf16, full_int8, kind):
    """48 one-token forwards queued back to back (one synchronisation at the
    end), each against the oracle. Each one-token engine's single launch
    orders its workgroups through counts and flags (row-dot engine) or
    partial slots holding a sentinel until written (split-K engine) that
    every launch must leave as it found them: a word left set would let the
    next launch read logits, hidden values or partials before they are
    written."""
    case = {"bf16": full_bf16, "int8": full_int8}[kind]
    xs = [syn.activations(1, 1280, seed=7000 + i) for i in range(48)]
    xd = [dev(x) for x in xs]
    yd = [torch.full_like(x, float("nan")) for x in xd]
    torch.cuda.synchronize()
    for x, y in zip(xd, yd):
        um.forward(ctx, case.layer, x, y, sync=False)
    ctx.synchronize()
    worst = 0.0
    for i, (x, y) in enumerate(zip(xs, yd)):
        got = y.cpu().numpy()
        ref, _ = oracle_ref(case, x)
        err = normwise(got, ref)
        worst = max(worst, err)
        assert np.all(np.isfinite(got)) and err <= FP32_TOL, (i, err)
    say(f"  {kind}: 48 queued one-token forwards, worst normwise {worst:.3e}")


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_decode_wait_bound(ctx, full_bf16, full_int8, kind):
    """The one-token engines' cross-workgroup waits are bounded. With the
    bound at 0 polls, the waits for the logits and for the hidden values
    (row-dot engine, BF16) or the down partials (split-K engine, INT8)
    cannot all be satisfied at their first poll: the forward reports
    Resource and the launch still ends. The words and partials it leaves
    set are reset with the error, so the same context at the default bound
    gives the right result again, twice in a row."""
    case = {"bf16": full_bf16, "int8": full_int8}[kind]
    say(f"decode wait bound 0, {kind}")
    x = syn.activations(1, 1280, seed=9100)
    ref, _ = oracle_ref(case, x)
    c2 = um.Context(0, 64 << 20)
    try:
        c2.set_wait_limit(0)
        xd, yd = dev(x), torch.empty((1, 1280), device="cuda")
        torch.cuda.synchronize()
        with pytest.raises(um.UocrError) as e:
            um.forward(c2, case.layer, xd, yd)
        assert e.value.status == um.RESOURCE
        c2.set_wait_limit(-1)
        for _ in range(2):
            um.forward(c2, case.layer, xd, yd)
            assert normwise(yd.cpu().numpy(), ref) <= FP32_TOL
    finally:
        c2.close()


# Stamps each role of the one-token engine writes, in the order it passes
# them (uocr_moe_trace::decode_stamps).
DECODE_STAMPS_SET = {"logit": (0, 1, 2, 3), "shared": (0, 3, 4), "routed": (0, 1, 2, 3, 4)}
# The output workgroups: down workgroups (BF16 layers), combine workgroups
# (INT8 overlays).
DECODE_OUTPUT_STAMPS = {"bf16": (0, 1, 3, 4, 5), "int8": (0, 1, 2, 3, 4, 5)}


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_decode_timeline_stamps(ctx, full_bf16, full_int8, kind):
    """The one-token engine's timeline: every workgroup of the launch
    writes its phase stamps (the device's real-time counter) in the order it
    passes them, leaves the other stamps and anything past its rows
    untouched, and the forward gives the same bits as without the
    timeline."""
    case = {"bf16": full_bf16, "int8": full_int8}[kind]
    rows = um.decode_stamp_rows(FULL["hidden"], FULL["inter"], FULL["experts"], FULL["shared"],
                                case.top_k)
    assert rows == {"logit": 8, "shared": 56, "routed": 168, "output": 160}
    n = sum(rows.values())
    x = syn.activations(1, 1280, seed=9300)
    xd = dev(x)
    y0, y1 = torch.empty_like(xd), torch.empty_like(xd)
    st = torch.full((n + 1, um.DECODE_STAMPS), -1, dtype=torch.int64, device="cuda")
    um.forward(ctx, case.layer, xd, y0)
    um.forward(ctx, case.layer, xd, y1, trace={"decode_stamps": st[:n]})
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
    a = st.cpu().numpy()
    assert (a[n] == -1).all()  # the row past the launch is never written
    r0 = 0
    for role in um.DECODE_ROLES:
        blk = a[r0:r0 + rows[role]]
        idx = DECODE_STAMPS_SET[role] if role != "output" else DECODE_OUTPUT_STAMPS[kind]
        unset = [j for j in range(um.DECODE_STAMPS) if j not in idx]
        assert (blk[:, list(idx)] > 0).all(), role
        assert (blk[:, unset] == -1).all(), role
        assert (np.diff(blk[:, list(idx)], axis=1) >= 0).all(), role
        r0 += rows[role]
    # One launch: its stamps span microseconds, not milliseconds (100 MHz).
    span = a[:n][a[:n] > 0].max() - a[:n, 0].min()
    say(f"  decode timeline {kind}: span {span / 100:.1f} us")
    assert 0 < span < 100_000


def _w8a8_trace(T, K, E):
    """Device buffers of uocr_w8a8_trace at the full layer shape."""
    S = FULL["inter"] * FULL["shared"]
    Hd, Id = FULL["hidden"], FULL["inter"]
    z = lambda *shape, dt=torch.int32: torch.full(shape, -7, dtype=dt, device="cuda")
    return {"gateup_sums": z(T * K, 2 * Id, Hd // 32), "down_sums": z(T * K, Hd, Id // 32),
            "hidden": z(T * K, Id, dt=torch.float32),
            "shared_gateup_sums": z(2 * S, Hd // 32), "shared_down_sums": z(Hd, S // 32),
            "shared_hidden": z(S, dt=torch.float32)}


def _check_single_groups(qd, x, offs, prow, g):
    """Every single-row group's W8A8 trace entries against the oracle's
    Int8Matrix::linear_dynamic_int8 (src/cpu/quantized.rs:190-198): gate/up
    block sums on the layer input row and down block sums on the GPU's own
    FP32 hidden row bit for bit (the oracle quantises that row again, so the
    quantisation is pinned as well), the hidden row within 1e-5 (FP32 sums
    of exact products in another order); the hidden rows of multi-row
    groups' positions untouched (-7). Returns the single-row expert ids."""
    Id = FULL["inter"]
    singles = []
    for e in range(FULL["experts"]):
        p0, p1 = offs[e], offs[e + 1]
        if p1 - p0 != 1:
            assert np.all(g["hidden"][p0:p1] == -7), (e, "multi-row position written")
            continue
        singles.append(e)
        p = p0
        xr = x[prow[p]].reshape(1, -1)
        _, gs = orc.int8_linear_dynamic(qd["gate"][0][e], qd["gate"][1][e], xr, with_block_sums=True)
        _, us = orc.int8_linear_dynamic(qd["up"][0][e], qd["up"][1][e], xr, with_block_sums=True)
        assert np.array_equal(g["gateup_sums"][p, :Id], gs), (e, "gate")
        assert np.array_equal(g["gateup_sums"][p, Id:], us), (e, "up")
        h = g["hidden"][p].reshape(1, -1)
        _, ds = orc.int8_linear_dynamic(qd["down"][0][e], qd["down"][1][e], h, with_block_sums=True)
        assert np.array_equal(g["down_sums"][p], ds), (e, "down")
        gy = orc.int8_linear_dynamic(qd["gate"][0][e], qd["gate"][1][e], xr)
        uy = orc.int8_linear_dynamic(qd["up"][0][e], qd["up"][1][e], xr)
        assert normwise(h, orc.silu(gy) * uy) < 1e-5, e
    return singles


@pytest.mark.parametrize("T,flags", [(1, 0), (8, 0), (17, 0), (1, um.FLAG_FORCE_GEMV)],
                         ids=["decode", "small-batch", "mfma-singles", "forced-small-batch"])
def test_w8a8_block_sums_bit_exact_in_layer(ctx, full_dynamic, T, flags):
    """The W8A8 dot that runs inside the layer (decode engine at T = 1, the
    small-batch engine at T <= 16 and for the single-row groups beside the
    MFMA GEMMs) stores its int32 block sums in the trace; each single-row
    group's sums equal the oracle's Int8Matrix::linear_dynamic_int8 block
    sums (src/cpu/quantized.rs:190-198) bit for bit: gate/up on the layer
    input row, down on the GPU's own FP32 hidden row (the oracle quantises
    it again, so the quantisation is pinned as well)."""
    K = full_dynamic.top_k
    x = syn.activations(T, FULL["hidden"], seed=900 + T)
    q8 = _w8a8_trace(T, K, FULL["experts"])
    tr = {"expert_offsets": torch.zeros(FULL["experts"] + 1, dtype=torch.int32, device="cuda"),
          "perm_rows": torch.zeros(T * K, dtype=torch.int32, device="cuda"),
          "w8a8": q8}
    xd = dev(x)
    yd = torch.empty_like(xd)
    um.forward(ctx, full_dynamic.layer, xd, yd, flags=flags, trace=tr)
    torch.cuda.synchronize()
    offs = tr["expert_offsets"].cpu().numpy()
    prow = tr["perm_rows"].cpu().numpy()
    g = {k: v.cpu().numpy() for k, v in q8.items()}
    qd = full_dynamic.orc.q
    Id = FULL["inter"]
    singles = _check_single_groups(qd, x, offs, prow, g)
    say(f"  W8A8 trace T={T} flags={flags}: {len(singles)} single-row groups")
    assert singles
    if T == 1:
        xr = x.reshape(1, -1)
        S = Id * FULL["shared"]
        _, gs = orc.int8_linear_dynamic(*qd["shared_gate"], xr, with_block_sums=True)
        _, us = orc.int8_linear_dynamic(*qd["shared_up"], xr, with_block_sums=True)
        assert np.array_equal(g["shared_gateup_sums"][:S], gs)
        assert np.array_equal(g["shared_gateup_sums"][S:], us)
        _, ds = orc.int8_linear_dynamic(*qd["shared_down"], g["shared_hidden"].reshape(1, -1),
                                        with_block_sums=True)
        assert np.array_equal(g["shared_down_sums"], ds)
    else:
        assert np.all(g["shared_gateup_sums"] == -7)  # untouched: the shared group has T rows


@pytest.mark.parametrize("T", [1, 2, 3])
def test_w8a8_singles_beside_forced_mfma_exact_scratch(full_dynamic, T):
    """The MFMA engine forced on 1-3 tokens of a DynamicActivations layer:
    every group has one row, so the small-batch engine's single-row pass
    runs every routed expert beside the MFMA kernels. Token t is built to
    select experts 58 - 6t .. 63 - 6t (ids far above 16 T), on a context
    whose scratch budget is exactly uocr_moe_scratch_bytes(cfg, T): the
    pass keeps its hidden rows by dispatched position inside that budget.
    Outputs against the oracle and the W8A8 trace bit for bit."""
    K, E, Hd = full_dynamic.top_k, FULL["experts"], FULL["hidden"]
    cfg = um.config(Hd, FULL["inter"], E, FULL["shared"], K, normalize=True)
    want = [list(range(58 - 6 * t, 64 - 6 * t)) for t in range(T)]
    r = syn.bf16_bits_to_f32(full_dynamic.w["router"]).astype(np.float64)
    noise = np.random.default_rng(31 + T).standard_normal((T, Hd)) * 0.05
    x = np.stack([r[w].sum(axis=0) / (r[w] ** 2).sum(axis=1).mean() * 2.0 for w in want])
    x = (x + noise).astype(np.float32)
    ref, rtr = oracle_ref(full_dynamic, x)
    for t in range(T):
        assert sorted(rtr.topk_ids[t].tolist()) == want[t], (t, rtr.topk_ids[t])
    exact = um.scratch_bytes(cfg, T)
    c = um.Context(0, exact)
    try:
        q8 = _w8a8_trace(T, K, E)
        tr = {"expert_offsets": torch.zeros(E + 1, dtype=torch.int32, device="cuda"),
              "perm_rows": torch.zeros(T * K, dtype=torch.int32, device="cuda"),
              "topk_ids": torch.zeros((T, K), dtype=torch.int32, device="cuda"),
              "w8a8": q8}
        xd = dev(x)
        yd = torch.full_like(xd, float("nan"))
        um.forward(c, full_dynamic.layer, xd, yd, flags=um.FLAG_FORCE_MFMA, trace=tr)
        torch.cuda.synchronize()
        y = yd.cpu().numpy()
        assert np.array_equal(tr["topk_ids"].cpu().numpy(), rtr.topk_ids)
        offs = tr["expert_offsets"].cpu().numpy()
        assert np.array_equal(offs, rtr.expert_offsets)
        g = {k: v.cpu().numpy() for k, v in q8.items()}
        singles = _check_single_groups(full_dynamic.orc.q, x, offs,
                                       tr["perm_rows"].cpu().numpy(), g)
        assert sorted(singles) == sorted(sum(want, []))
        err = normwise(y, ref)
        say(f"  forced MFMA W8A8 T={T}, scratch {exact} B: normwise {err:.3e}, "
            f"experts {min(singles)}..{max(singles)}")
        assert err <= FP32_TOL, err
    finally:
        c.close()


def test_deterministic_and_row_independent(ctx, full_bf16):
    say("determinism and row independence, T=256")
    x = syn.activations(256, 1280, seed=7)
    y1, _ = full_bf16.run(ctx, x)
    y2, _ = full_bf16.run(ctx, x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    rows = [0, 17, 255]
    ref = orc.moe_experts(full_bf16.orc, x[rows])
    assert normwise(y1[rows], ref) <= FP32_TOL


def test_layer_errors(ctx):
    say("layer errors: non-finite input, scratch budget, overlay")
    case = Case(ctx, SMALL, 4, seed=5)
    x = syn.activations(3, SMALL["hidden"], seed=6)
    x[1, 2] = np.nan
    with pytest.raises(um.UocrError) as e:
        case.run(ctx, x)
    assert e.value.status == um.NUMERICAL
    # The context recovers after the error.
    case.run(ctx, syn.activations(3, SMALL["hidden"], seed=6))
    tiny = um.Context(0, 4096)
    xd = dev(syn.activations(64, SMALL["hidden"], seed=6))
    with pytest.raises(um.UocrError) as e:
        um.forward(tiny, case.layer, xd, torch.empty_like(xd))
    assert e.value.status == um.RESOURCE
    tiny.close()
    with pytest.raises(um.UocrError) as e:
        case.layer.attach_int8(ctx, {}, um.MEMORY_HOST, um.QUANT_DYNAMIC)
    assert e.value.status == um.FORMAT
    q = syn.int8_overlay(seed=9, **SMALL)
    qb = dict(q)
    g, s = q["gate"]
    g = g.copy()
    g[0, 0, 0] = -128
    qb["gate"] = (g, s)
    with pytest.raises(um.UocrError) as e:
        case.layer.attach_int8(ctx, qb, um.MEMORY_HOST, um.QUANT_WEIGHTS_ONLY)
    assert e.value.status == um.FORMAT
    assert case.layer.precision == "bf16_weights_fp32"


# ----------------------------------------------------------- engine choice

BF16_TOL = 2e-2


@pytest.mark.parametrize("T", [1, 17, 129, 300])
def test_small_layer_engines(ctx, T):
    """Both engines at every size: GEMV (FP32) and MFMA with FP32-class
    (hi+lo bf16) and BF16 activations."""
    case = Case(ctx, SMALL, 4, seed=40 + T, normalize=True)
    x = syn.activations(T, SMALL["hidden"], seed=50 + T)
    say(f"small engines T={T}: gemv")
    check_layer(case, ctx, x, flags=um.FLAG_FORCE_GEMV)
    say(f"small engines T={T}: mfma fp32-class")
    check_layer(case, ctx, x, flags=um.FLAG_FORCE_MFMA)
    say(f"small engines T={T}: mfma bf16 activations")
    check_layer(case, ctx, x, tol=BF16_TOL,
                flags=um.FLAG_FORCE_MFMA | um.FLAG_BF16_ACTIVATIONS)


@pytest.mark.parametrize("T", [64, 512])
def test_full_bf16_mfma(ctx, full_bf16, T):
    x = syn.activations(T, 1280, seed=600 + T)
    say(f"full BF16 MFMA fp32-class T={T}")
    check_layer(full_bf16, ctx, x, flags=um.FLAG_FORCE_MFMA)
    say(f"full BF16 MFMA bf16 activations T={T}")
    check_layer(full_bf16, ctx, x, tol=BF16_TOL,
                flags=um.FLAG_FORCE_MFMA | um.FLAG_BF16_ACTIVATIONS)


@pytest.mark.parametrize("T", [17, 64, 512])
def test_int8_mfma(ctx, full_int8, full_dynamic, T):
    """INT8 overlays on the MFMA engine: int8 rows (exact in bf16) and block
    scales are streamed; each 32-deep block's partial product with the
    activation planes (hi + lo for the FP32 class, hi for BF16 activations)
    is scaled by its block scale into the f32 accumulator. 64-row tiles run
    as 64 x 512 items (T = 512 puts ~48 rows in each expert). Under
    DynamicActivations the groups of one row take the W8A8 path
    (src/decoder/mod.rs:103-104); T = 17 and 64 leave several such groups
    among 64 experts."""
    x = syn.activations(T, 1280, seed=700 + T)
    for case, name in ((full_int8, "weight-only"), (full_dynamic, "dynamic")):
        say(f"INT8 MFMA {name} T={T}")
        check_layer(case, ctx, x)
        if T == 64:
            say(f"INT8 MFMA {name} T={T} bf16 activations")
            check_layer(case, ctx, x, tol=BF16_TOL, flags=um.FLAG_BF16_ACTIVATIONS)
            say(f"INT8 small-batch engine forced {name} T={T}")
            check_layer(case, ctx, x, flags=um.FLAG_FORCE_GEMV)
    if T == 64:
        _, tr = full_dynamic.run(ctx, x)
        counts = np.diff(tr["expert_offsets"])
        assert (counts == 1).any(), counts  # the W8A8 single-row path ran


@pytest.mark.parametrize("kind", ["bf16", "int8", "w8a8"])
def test_one_stream_matches_two_streams(ctx, full_bf16, full_int8, full_dynamic, kind):
    """Up to 2048 tokens the shared expert's GEMMs run on a second stream
    after a split of the input into bf16 planes; on one stream (phase
    timing on) the router writes those planes itself. Under
    DynamicActivations the single-row pass runs on the main stream after
    the dispatch, before the routed GEMMs, with its hidden rows in its own
    scratch rows by dispatched position (24 tokens leave 15 groups of one
    row). Same bits either way, in both activation classes."""
    case = {"bf16": full_bf16, "int8": full_int8, "w8a8": full_dynamic}[kind]
    T = 24 if kind == "w8a8" else 512
    x = syn.activations(T, 1280, seed=811)
    for flags, name in ((0, "fp32-class"), (um.FLAG_BF16_ACTIVATIONS, "bf16 activations")):
        say(f"{kind} T={T} {name}: two streams vs one")
        y2, tr = case.run(ctx, x, flags=um.FLAG_FORCE_MFMA | flags)
        if kind == "w8a8":
            assert (np.diff(tr["expert_offsets"]) == 1).sum() == 15
        ctx.set_timing("all")
        try:
            y1, _ = case.run(ctx, x, flags=um.FLAG_FORCE_MFMA | flags)
        finally:
            ctx.set_timing(())
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), name


@pytest.fixture(scope="module")
def hot_bf16(ctx):
    hot = syn.route_profile(syn.hot_share(FULL["experts"], 6, 8, 0.8), 6)
    return Case(ctx, FULL, 6, seed=41, router_scale=hot)


def test_mfma_hot_experts(ctx, hot_bf16):
    """Skewed routing (80% of assignments on 8 experts): hot experts span
    several 256-row tiles whose last tile is partial, cold experts fill one
    small tile. Rows are independent, so a sample of rows is checked against
    the oracle."""
    T = 1536
    x = syn.activations(T, 1280, seed=77)
    rows = np.sort(np.random.default_rng(5).choice(T, 40, replace=False))
    ref, rtr = orc.moe_experts(hot_bf16.orc, x[rows], trace=True)
    for flags, tol in ((0, FP32_TOL), (um.FLAG_BF16_ACTIVATIONS, BF16_TOL)):
        say(f"hot-expert MFMA T={T} flags={flags}")
        y, tr = hot_bf16.run(ctx, x, flags)
        counts = np.diff(tr["expert_offsets"])
        tail = counts % 256
        assert (counts > 256).any()
        assert ((tail > 128) & (counts > 256)).any() and ((tail > 0) & (tail <= 128)).any()
        assert np.all(np.isfinite(y))
        keep = []
        for i, t in enumerate(rows):
            a, b = set(rtr.topk_ids[i].tolist()), set(tr["topk_ids"][t].tolist())
            if a == b:
                keep.append(i)
                continue
            # A differing selection must be a logit tie within 1e-6.
            kth = np.sort(rtr.logits[i])[::-1][hot_bf16.top_k - 1]
            for e in a ^ b:
                assert abs(float(rtr.logits[i][e]) - float(kth)) <= TIE, (t, e)
        err = normwise(y[rows[keep]], ref[keep])
        say(f"  normwise={err:.3e}")
        assert err <= tol, err


# ------------------------------------------------------------ block stack

def _stack(ctx, n, quant=orc.QUANT_NONE):
    """n SMALL layers with distinct weights and non-trivial norm weights."""
    cases, norms = [], []
    for l in range(n):
        c = Case(ctx, SMALL, 4, seed=900 + 7 * l, quant=quant, normalize=True)
        nw = (0.75 + 0.5 * np.sin(np.arange(SMALL["hidden"]) * (0.3 + 0.1 * l))).astype(np.float32)
        nw = orc.bf16_to_f32(orc.f32_to_bf16(nw))
        c.w["norm_weight"] = orc.f32_to_bf16(nw).view(np.uint16)
        cfg = um.config(SMALL["hidden"], SMALL["inter"], SMALL["experts"], SMALL["shared"], 4,
                        normalize=True)
        c.layer = um.MoeLayer(ctx, cfg, c.w, um.MEMORY_HOST)
        if quant != orc.QUANT_NONE:
            c.layer.attach_int8(ctx, c.orc.q, um.MEMORY_HOST, quant)
        cases.append(c)
        norms.append(nw)
    return cases, norms


def _stack_ref(cases, norms, x, eps=1e-6):
    """Oracle stack, and the tokens whose routing has a near-tie at some layer."""
    near = np.zeros(x.shape[0], bool)
    for c, nw in zip(cases, norms):
        n = orc.rms_norm(x, nw, eps)
        out, tr = orc.moe_experts(c.orc, n, trace=True)
        srt = np.sort(tr.logits, axis=1)[:, ::-1]
        near |= (srt[:, c.top_k - 1] - srt[:, c.top_k]) < 1e-5
        x = x + out
    return x, near


@pytest.mark.parametrize("quant", [orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY])
@pytest.mark.parametrize("T", [1, 8, 40, 300])
def test_block_stack(ctx, T, quant):
    """uocr_moe_block_forward over 3 layers (RMSNorm of each layer fused into
    the previous layer's combine, with the MFMA engine's bf16 planes) against
    the oracle's moe_block chain."""
    cases, norms = _stack(ctx, 3, quant)
    x = syn.activations(T, SMALL["hidden"], seed=1000 + T)
    ref, near = _stack_ref(cases, norms, x)
    keep = ~near
    flag_sets = [(0, FP32_TOL)]
    if quant == orc.QUANT_NONE and T > 16:
        flag_sets.append((um.FLAG_BF16_ACTIVATIONS, BF16_TOL))
    for flags, tol in flag_sets:
        say(f"block stack T={T} quant={quant} flags={flags}")
        xd = dev(x)
        yd = torch.full_like(xd, float("nan"))
        um.block_forward(ctx, [c.layer for c in cases], xd, yd, flags=flags)
        y = yd.cpu().numpy()
        assert np.all(np.isfinite(y))
        err = normwise(y[keep], ref[keep])
        say(f"  normwise={err:.3e} (near-ties {int(near.sum())})")
        assert err <= tol, err


@pytest.mark.parametrize("H", [128, 1280, 1536, 2048])
@pytest.mark.parametrize("T", [8, 40])
def test_fused_norm_bits(ctx, H, T):
    """The next layer's RMSNorm fused into a combine gives the standalone
    norm's bits: a 2-layer block forward equals two 1-layer block forwards
    (each with a standalone first norm), bit for bit, at widths that take
    the one-row-per-wave form (<= 1280) and the one-row-per-workgroup form."""
    shape = dict(hidden=H, inter=64, experts=16, shared=2)
    layers = []
    for l in range(2):
        c = Case(ctx, shape, 4, seed=1500 + 11 * l + H, normalize=True)
        nw = (0.75 + 0.5 * np.sin(np.arange(H) * (0.2 + 0.1 * l))).astype(np.float32)
        c.w["norm_weight"] = orc.f32_to_bf16(nw).view(np.uint16)
        cfg = um.config(H, shape["inter"], shape["experts"], shape["shared"], 4, normalize=True)
        c.layer = um.MoeLayer(ctx, cfg, c.w, um.MEMORY_HOST)
        layers.append(c.layer)
    say(f"fused norm bits H={H} T={T}")
    x = dev(syn.activations(T, H, seed=77 + T))
    both = torch.empty_like(x)
    um.block_forward(ctx, layers, x, both)
    one = torch.empty_like(x)
    two = torch.empty_like(x)
    um.block_forward(ctx, layers[:1], x, one)
    um.block_forward(ctx, layers[1:], one, two)
    assert np.array_equal(both.cpu().numpy().view(np.uint32), two.cpu().numpy().view(np.uint32))


# ------------------------------------------------------ vocabulary projection

@pytest.mark.parametrize("V,H", [(1000, 1280), (4099, 1280), (517, 2048), (300, 192),
                                 (257, 96)])
@pytest.mark.parametrize("kind", ["bf16", "int8", "w8a8"])
def test_lm_head(ctx, V, H, kind):
    """Decoder::logits: RMSNorm of the last hidden row, then the projection
    (src/decoder/mod.rs:99-112, 367-379). Widths that are multiples of 64 up
    to 2048 take the one-launch kernel; 96 takes the operator fallback. FP32
    accumulation order differs from the oracle's: 1e-5 normwise; W8A8 also
    quantises the normalised row, where a 1-ulp difference in the norm can
    move one int8 by one step: 3e-3."""
    rng = np.random.default_rng(V + H)
    say(f"lm_head V={V} H={H} {kind}")
    hidden = rng.standard_normal((3, H), dtype=np.float32)
    norm = orc.bf16_to_f32(orc.f32_to_bf16(0.5 + rng.random(H, dtype=np.float32)))
    n = orc.rms_norm(hidden[-1:], norm, 1e-6)
    if kind == "bf16":
        w = orc.f32_to_bf16(rng.standard_normal((V, H), dtype=np.float32) * 0.05)
        ref = orc.linear_weight_bf16(n, w)
        head = um.LmHead(ctx, dev(norm), 1e-6, weight=dev(w.view(np.int16)), where=um.MEMORY_DEVICE)
        tol = 1e-5
    else:
        q = rng.integers(-127, 128, (V, H), dtype=np.int8)
        sc = (rng.random((V, H // 32), dtype=np.float32) * 0.002 + 0.001).astype(np.float32)
        mode = um.QUANT_WEIGHTS_ONLY if kind == "int8" else um.QUANT_DYNAMIC
        ref = orc.int8_linear(q, sc, n) if kind == "int8" else orc.int8_linear_dynamic(q, sc, n)
        head = um.LmHead(ctx, dev(norm), 1e-6, q=dev(q), scales=dev(sc), mode=mode,
                         where=um.MEMORY_DEVICE)
        tol = 1e-5 if kind == "int8" else 3e-3
    assert head.precision == {"bf16": "bf16_weights_fp32", "int8": "int8_weights_fp32",
                              "w8a8": "int8_weights_dynamic_activations"}[kind]
    out = torch.full((V,), float("nan"), device="cuda")
    head.logits(ctx, dev(hidden), out)
    got = out.cpu().numpy().reshape(1, V)
    assert np.all(np.isfinite(got))
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    say(f"  normwise={err:.3e}")
    assert err <= tol, err
    if V == 1000 and kind == "bf16":
        bad = hidden.copy()
        bad[-1, 3] = np.inf
        with pytest.raises(um.UocrError) as e:
            head.logits(ctx, dev(bad), out)
        assert e.value.status == um.NUMERICAL
        with pytest.raises(um.UocrError) as e:
            head.logits(ctx, dev(hidden)[:0], out)
        assert e.value.status == um.SHAPE
    head.close()
