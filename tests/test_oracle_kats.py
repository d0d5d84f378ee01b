"""Pins the CPU oracle to the reference's own known-answer tests for the MoE
path, plus closed forms. Each test names the reference test it ports."""
import math

import numpy as np
import pytest

import oracle as orc


def test_route_kat():
    # tests/moe.rs:4-13
    assert orc.route([0.0, 0.0, 0.0, 0.0], 2, False, 1.0) == [(0, 0.25), (1, 0.25)]
    assert orc.route([0.0, 0.0, 0.0, 0.0], 2, True, 2.0) == [(0, 1.0), (1, 1.0)]
    with pytest.raises(orc.OracleError) as e:
        orc.route([0.0, float("nan")], 1, False, 1.0)
    assert e.value.status == orc.NUMERICAL
    with pytest.raises(orc.OracleError) as e:
        orc.route([0.0], 2, False, 1.0)
    assert e.value.status == orc.SHAPE


def test_route_argument_rules():
    # src/decoder/moe.rs:13-15: count 0, count > len, scale <= 0 or non-finite.
    for count, scale in [(0, 1.0), (3, 1.0), (1, 0.0), (1, -1.0), (1, float("inf")),
                         (1, float("nan"))]:
        with pytest.raises(orc.OracleError) as e:
            orc.route([0.0, 1.0], count, False, scale)
        assert e.value.status == orc.SHAPE


def test_route_order_is_probability_then_id():
    # Sort key (p desc, id asc) of src/decoder/moe.rs:19 — brute force on ties.
    logits = [1.0, 3.0, 3.0, 2.0, 3.0]
    got = [i for i, _ in orc.route(logits, 5, False, 1.0)]
    assert got == [1, 2, 4, 3, 0]


def test_route_normalised_weights_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(50):
        logits = rng.standard_normal(64).astype(np.float32)
        ids, w = orc.route_arrays(logits, 6, True, 2.5)
        p = np.exp(logits.astype(np.float64) - logits.max())
        p /= p.sum()
        order = sorted(range(64), key=lambda i: (-p[i], i))[:6]
        assert list(ids) == order
        expect = p[order] / p[order].sum() * 2.5
        np.testing.assert_allclose(w, expect, rtol=1e-5)


def test_linear_kat():
    # tests/ops.rs:10-20
    x = np.array([[1, 2, 3], [-1, 0, 2]], np.float32)
    w = np.array([[1, 0, -1], [2, 1, 0]], np.float32)
    y = orc.linear(x, w, bias=np.array([1, -1], np.float32))
    assert y.ravel().tolist() == [-1.0, 3.0, -2.0, -3.0]


def test_softmax_kats():
    # tests/ops.rs:33-40
    assert orc.softmax([1000.0, 1000.0, -1000.0]).tolist() == [0.5, 0.5, 0.0]
    for bad in ([float("nan"), 0.0], [float("-inf")] * 2, [], [float("inf")]):
        with pytest.raises(orc.OracleError) as e:
            orc.softmax(bad)
        assert e.value.status == orc.NUMERICAL


def test_softmax_matches_f64_oracle():
    # tests/ops.rs:101-132 (Scalar backend).
    for n in [1, 3, 17, 196, 4096]:
        x = np.array([-np.inf if i % 7 == 3 else 1000.0 + math.sin(i * 0.37) * 30.0
                      for i in range(n)], np.float32)
        m = float(np.max(x))
        e = np.exp(x.astype(np.float64) - m)
        want = e / e.sum()
        got = orc.softmax(x)
        assert np.all(np.abs(got.astype(np.float64) - want) < 2e-6)


def test_rms_norm_kat():
    # tests/ops.rs:42-51
    y = orc.rms_norm(np.array([[1.0, 3.0]], np.float32), np.array([1.0, 1.0], np.float32), 1e-6)
    assert abs(y[0, 0] - 0.44721355) < 1e-6
    assert abs(y[0, 1] - 1.3416406) < 1e-6
    with pytest.raises(orc.OracleError) as e:
        orc.rms_norm(np.array([[1.0, np.inf]], np.float32), np.ones(2, np.float32), 1e-6)
    assert e.value.status == orc.NUMERICAL


def test_silu_kat():
    # tests/ops.rs:74-84
    y = orc.silu(np.array([-1.0, 0.0, 1.0], np.float32))
    for a, b in zip(y, [-0.26894143, 0.0, 0.7310586]):
        assert abs(a - b) < 1e-6


def test_bf16_widening_and_encode():
    # src/checkpoint.rs:79-85 widening is exact; half's RNE encode.
    bits = np.array([0x3F80, 0xBF80, 0x0000, 0x8000, 0x7F80, 0x4049], np.uint16)
    assert orc.bf16_to_f32(bits).tolist() == [1.0, -1.0, 0.0, -0.0, float("inf"), 3.140625]
    for b in bits:
        assert orc.lib().orc_bf16_to_f32(int(b)) == orc.bf16_to_f32(np.array([b]))[0] or \
            math.isinf(orc.bf16_to_f32(np.array([b]))[0])
    # Ties to even: 1 + 2^-8 sits halfway between 1 and 1 + 2^-7.
    assert orc.f32_to_bf16(np.array([1.0 + 2 ** -8], np.float32))[0] == 0x3F80
    assert orc.f32_to_bf16(np.array([1.0 + 3 * 2 ** -8], np.float32))[0] == 0x3F82
    for v in [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -7.3, 1e-30]:
        a = orc.lib().orc_f32_to_bf16(v)
        assert a == orc.f32_to_bf16(np.array([v], np.float32))[0]


def test_bf16_linear_weight_matches_f32_linear():
    # tests/weights.rs:9-50: BF16 view vs the widened F32 linear, odd rows, tails.
    for rows in [37, 1025]:
        cols = 131
        w = np.array([((i % 29) - 14) / 16 for i in range(rows * cols)], np.float32)
        w = w.reshape(rows, cols)
        bits = orc.f32_to_bf16(w)
        for batch in [1, 3]:
            x = np.array([((i % 13) - 6) / 8 for i in range(batch * cols)], np.float32)
            x = x.reshape(batch, cols)
            want = orc.linear(x, w)
            for threads in [1, 3]:
                got = orc.linear_weight_bf16(x, bits, threads=threads)
                assert np.all(np.abs(got - want) < 1e-5)


def test_int8_dequantize_bit_exact():
    # tests/quantized.rs:6-29
    for cols in [1, 31, 32, 33, 513, 1280]:
        rows = 5
        q = np.array([((i % 255) - 127) for i in range(rows * cols)], np.int8).reshape(rows, cols)
        nb = (cols + 31) // 32
        s = np.array([[0.0, -0.0, 0.1234567, 1e-20, 1e20][i % 5] for i in range(rows * nb)],
                     np.float32).reshape(rows, nb)
        assert orc.int8_check(rows, cols, q, s) == orc.OK
        got = orc.int8_dequantize(q, s)
        want = (q.astype(np.float64) * np.repeat(s, 32, axis=1)[:, :cols].astype(np.float64))
        want = want.astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_int8_roundtrip_and_linear():
    # tests/quantized.rs:31-73
    for cols in [1, 31, 32, 33, 131, 513]:
        rows = 257 if cols == 513 else 7
        vals = np.array([0.0 if i // cols == 0 else math.sin(np.float32(i) * np.float32(0.37)) * 3
                         for i in range(rows * cols)], np.float32).reshape(rows, cols)
        q, s = orc.int8_quantize(vals)
        restored = orc.int8_dequantize(q, s)
        assert np.all(np.abs(restored - vals) <= 3.0 / 254.0 + 1e-6)
        assert np.all(restored[0] == 0.0)
        for batch in [1, 3]:
            x = np.cos(np.arange(batch * cols, dtype=np.float32) * np.float32(0.13))
            x = x.astype(np.float32).reshape(batch, cols)
            want = x.astype(np.float64) @ restored.astype(np.float64).T
            for threads in [1, 3]:
                got = orc.int8_linear(q, s, x, threads=threads)
                assert np.all(np.abs(got - want) < 2e-5)


def test_int8_invalid_storage():
    # tests/quantized.rs:74-87
    assert orc.int8_check(1, 33, np.zeros(33, np.int8), np.array([1.0], np.float32)) == orc.SHAPE
    assert orc.int8_check(1, 1, np.zeros(1, np.int8), np.array([np.nan], np.float32)) == \
        orc.NUMERICAL
    assert orc.int8_check(1, 1, np.zeros(1, np.int8), np.array([-1.0], np.float32)) == \
        orc.NUMERICAL
    assert orc.int8_check(0, 1, np.zeros(0, np.int8), np.zeros(0, np.float32)) == orc.SHAPE
    with pytest.raises(orc.OracleError) as e:
        orc.int8_quantize(np.array([[np.inf]], np.float32))
    assert e.value.status == orc.NUMERICAL


def test_dynamic_int8_matches_explicit_quantized_reference():
    # tests/quantized.rs:89-120, plus the exact i32 block sums by brute force.
    for cols in [1, 15, 31, 32, 33, 131, 1280]:
        rows = 129 if cols == 1280 else 9
        m = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.41))
        q, s = orc.int8_quantize(m.astype(np.float32).reshape(rows, cols))
        x = (np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.17)) * 2).astype(np.float32)
        xq, xs = orc.int8_quantize(x.reshape(1, cols))
        rounded = orc.int8_dequantize(xq, xs)
        w = orc.int8_dequantize(q, s)
        y, sums = orc.int8_linear_dynamic(q, s, x.reshape(1, cols), threads=3,
                                          with_block_sums=True)
        want = w.astype(np.float64) @ rounded.astype(np.float64).ravel()
        assert np.all(np.abs(y.ravel() - want) < 2e-4), cols
        nb = (cols + 31) // 32
        pad = nb * 32 - cols
        qi = np.pad(q.astype(np.int64), ((0, 0), (0, pad))).reshape(rows, nb, 32)
        xi = np.pad(xq.astype(np.int64).ravel(), (0, pad)).reshape(nb, 32)
        assert np.array_equal(sums, (qi * xi[None]).sum(axis=2))


def test_overlay_linear_kat():
    # tests/quantized_loader.rs:36-48: int8 [1,-2], scale 1, x [3,4] -> [-5].
    y = orc.int8_linear(np.array([[1, -2]], np.int8), np.array([[1.0]], np.float32),
                        np.array([[3.0, 4.0]], np.float32))
    assert y.ravel().tolist() == [-5.0]


def test_python_quantizer_kat():
    # tests/python/test_quantize.py:8-16 (the producer uses the same rule).
    x = (np.arange(105, dtype=np.float32).reshape(3, 35) / 37 - 1).astype(np.float32)
    x[0] = 0
    q, s = orc.int8_quantize(x)
    assert s.shape == (3, 2)
    decoded = q.astype(np.float32) * np.repeat(s, 32, axis=1)[:, :35]
    assert np.all(np.abs(decoded - x) <= np.repeat(s / 2, 32, axis=1)[:, :35] + 1e-6)
    assert np.all(q[0] == 0) and np.all(s[0] == 0)
