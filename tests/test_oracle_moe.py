"""Pins the oracle's MoE-layer composition (Decoder::experts,
src/decoder/mod.rs:99-220) against an independent float64 restatement on
small shapes, and against the reference's own invariants: decode-task
parallelism and thread count never change bits (tests/decoder.rs:12-32),
rows are independent, dispatch order is (expert, row)."""
import numpy as np
import pytest

import oracle as orc
from uocr_moe import synthetic as syn

SMALL = dict(hidden=128, inter=64, experts=16, shared=2)


def small_layer(seed=0, top_k=4, normalize=True, scale=1.0, quant=orc.QUANT_NONE):
    w = syn.moe_weights(seed=seed, **SMALL)
    L = orc.MoeWeights(hidden=SMALL["hidden"], inter=SMALL["inter"], n_experts=SMALL["experts"],
                       top_k=top_k, n_shared=SMALL["shared"], normalize=normalize, scale=scale,
                       router=w["router"], gate=w["gate"], up=w["up"], down=w["down"],
                       shared_gate=w["shared_gate"], shared_up=w["shared_up"],
                       shared_down=w["shared_down"])
    if quant != orc.QUANT_NONE:
        L.quant_mode = quant
        L.q = syn.int8_overlay(seed=seed + 1, **SMALL)
    return L


def f64_ffn(x, g, u, d):
    a = x @ g.T
    b = x @ u.T
    h = a / (1 + np.exp(-a)) * b
    return h @ d.T


def f64_experts(L, x, weights_of):
    """Independent float64 MoE: softmax top-k by (p desc, id asc), shared +
    sum p * expert over the selected experts."""
    x = x.astype(np.float64)
    router = orc.bf16_to_f32(L.router).astype(np.float64)
    logits = x @ router.T
    out = f64_ffn(x, *weights_of("shared"))
    for t in range(x.shape[0]):
        p = np.exp(logits[t] - logits[t].max())
        p /= p.sum()
        order = sorted(range(L.n_experts), key=lambda i: (-p[i], i))[:L.top_k]
        den = p[order].sum() if L.normalize else 1.0
        for e in order:
            out[t] += p[e] / den * L.scale * f64_ffn(x[t:t + 1], *weights_of(e))[0]
    return out


def bf16_weights_of(L):
    def get(e):
        if e == "shared":
            return [orc.bf16_to_f32(a).astype(np.float64)
                    for a in (L.shared_gate, L.shared_up, L.shared_down)]
        return [orc.bf16_to_f32(a[e]).astype(np.float64) for a in (L.gate, L.up, L.down)]
    return get


def int8_weights_of(L):
    def deq(name, e=None):
        q, s = L.q[name]
        if e is not None:
            q, s = q[e], s[e]
        return orc.int8_dequantize(q, s).astype(np.float64)

    def get(e):
        if e == "shared":
            return [deq(n) for n in ("shared_gate", "shared_up", "shared_down")]
        return [deq(n, e) for n in ("gate", "up", "down")]
    return get


def normwise(a, b):
    """max over rows of ||a - b||_inf / ||b||_inf."""
    num = np.abs(a - b).max(axis=1)
    den = np.maximum(np.abs(b).max(axis=1), 1e-30)
    return float((num / den).max())


@pytest.mark.parametrize("T", [1, 5, 33])
@pytest.mark.parametrize("normalize", [True, False])
def test_bf16_layer_matches_float64(T, normalize):
    L = small_layer(seed=T, normalize=normalize, scale=1.5)
    x = syn.activations(T, SMALL["hidden"], seed=100 + T)
    y = orc.moe_experts(L, x)
    want = f64_experts(L, x, bf16_weights_of(L))
    assert normwise(y, want) < 1e-5


def test_int8_weights_only_layer_matches_float64():
    L = small_layer(seed=7, quant=orc.QUANT_WEIGHTS_ONLY)
    x = syn.activations(20, SMALL["hidden"], seed=8)
    y = orc.moe_experts(L, x)
    assert normwise(y, f64_experts(L, x, int8_weights_of(L))) < 1e-5


def test_dynamic_mode_quantises_only_single_row_groups():
    """DynamicActivations int8-rounds a projection input only when its
    group has one row (src/decoder/mod.rs:103-104). With T=1 every group has
    one row: the result differs from weights-only by the activation
    rounding; with a 2-row batch where both rows pick the same experts,
    nothing is rounded and the result equals weights-only bit for bit."""
    Lw = small_layer(seed=9, quant=orc.QUANT_WEIGHTS_ONLY)
    Ld = small_layer(seed=9, quant=orc.QUANT_DYNAMIC)
    x1 = syn.activations(1, SMALL["hidden"], seed=10)
    yw, yd = orc.moe_experts(Lw, x1), orc.moe_experts(Ld, x1)
    assert not np.array_equal(yw, yd)
    assert normwise(yd, yw) < 0.05
    x2 = np.concatenate([x1, x1])
    assert np.array_equal(orc.moe_experts(Ld, x2), orc.moe_experts(Lw, x2))


def test_decode_tasks_and_threads_keep_bits():
    # tests/decoder.rs:12-32: 1 thread, 8 threads, 8 threads + small scratch.
    for quant in (orc.QUANT_NONE, orc.QUANT_WEIGHTS_ONLY, orc.QUANT_DYNAMIC):
        L = small_layer(seed=3, quant=quant)
        x = syn.activations(1, SMALL["hidden"], seed=4)
        a = orc.moe_experts(L, x, threads=1)
        b = orc.moe_experts(L, x, threads=8)
        c = orc.moe_experts(L, x, threads=8, scratch_limit=64 * 1024)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


def test_rows_are_independent_and_permutable():
    L = small_layer(seed=11)
    x = syn.activations(24, SMALL["hidden"], seed=12)
    y = orc.moe_experts(L, x)
    perm = np.random.default_rng(0).permutation(24)
    assert np.array_equal(orc.moe_experts(L, x[perm]), y[perm])
    assert np.array_equal(orc.moe_experts(L, x[5:6]), y[5:6])


def test_dispatch_trace_is_stable_expert_major():
    L = small_layer(seed=13)
    T = 40
    x = syn.activations(T, SMALL["hidden"], seed=14)
    _, tr = orc.moe_experts(L, x, trace=True)
    E, K = L.n_experts, L.top_k
    counts = np.bincount(tr.topk_ids.ravel(), minlength=E)
    assert np.array_equal(tr.expert_offsets, np.concatenate([[0], np.cumsum(counts)]))
    want = sorted((int(e), t, float(w)) for t in range(T)
                  for e, w in zip(tr.topk_ids[t], tr.topk_weights[t]))
    assert [r for _, r, _ in want] == tr.perm_rows.tolist()
    assert [w for _, _, w in want] == tr.perm_weights.tolist()
    for t in range(T):
        ids, w = orc.route_arrays(tr.logits[t], K, True, 1.0)
        assert np.array_equal(ids, tr.topk_ids[t])
        assert np.array_equal(w, tr.topk_weights[t])


def test_block_is_residual_plus_experts_of_norm():
    L = small_layer(seed=15)
    x = syn.activations(6, SMALL["hidden"], seed=16)
    nw = np.ones(SMALL["hidden"], np.float32)
    y = orc.moe_block(L, nw, 1e-6, x)
    n = orc.rms_norm(x, nw, 1e-6)
    assert np.array_equal(y, x + orc.moe_experts(L, n))


def test_errors():
    L = small_layer(seed=17)
    x = syn.activations(2, SMALL["hidden"], seed=18)
    with pytest.raises(orc.OracleError) as e:
        orc.moe_experts(L, x, scratch_limit=4)
    assert e.value.status == orc.RESOURCE
    bad = x.copy()
    bad[1, 3] = np.nan
    with pytest.raises(orc.OracleError) as e:
        orc.moe_experts(L, bad)
    assert e.value.status == orc.NUMERICAL
    Ld = small_layer(seed=17)
    Ld.quant_mode = orc.QUANT_DYNAMIC  # no overlay attached
    with pytest.raises(orc.OracleError) as e:
        orc.moe_experts(Ld, x)
    assert e.value.status == orc.FORMAT


def test_row_parallel_block_is_bit_identical():
    """orc_moe_block_rows (the CPU-baseline timing aid that splits the
    prefill GEMM's rows over threads) returns the serial block's bits."""
    w = small_layer(seed=31)
    x = syn.activations(37, w.hidden, seed=32)
    nw = np.linspace(0.5, 1.5, w.hidden).astype(np.float32)
    a = orc.moe_block(w, nw, 1e-6, x)
    b = orc.moe_block(w, nw, 1e-6, x, row_threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("T", [1, 37])
def test_threaded_experts_are_bit_identical(T):
    """orc_moe_experts_threads (pool workers plus the prefill row split, the
    CPU-baseline timing aid) returns the serial experts' bits, for BF16 and
    for an INT8 overlay in DynamicActivations mode."""
    w = small_layer(seed=33)
    x = syn.activations(T, w.hidden, seed=34)
    a = orc.moe_experts(w, x)
    b = orc.moe_experts_threads(w, x, threads=4, row_threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    q = syn.int8_overlay(hidden=w.hidden, inter=w.inter, experts=w.n_experts, shared=w.n_shared,
                         seed=35)
    w.quant_mode = orc.QUANT_DYNAMIC
    w.q = q
    a = orc.moe_experts(w, x)
    b = orc.moe_experts_threads(w, x, threads=4, row_threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
