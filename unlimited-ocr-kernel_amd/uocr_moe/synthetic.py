"""Seeded synthetic MoE-layer workloads (no checkpoints are available offline).

Weights follow the benchmark definitions: BF16 N(0, 0.02) rounded to nearest
even; INT8 overlay int8 uniform in [-127, 127] with per-32-block scales
|N(0.002, 0.0005)|; activations N(0, 1). The router has no bias
(src/decoder/mod.rs:126 passes bias None), so expert popularity is shaped by
scaling router rows: a larger row norm gives an expert larger logits more
often. `route_profile` calibrates those scales by Monte Carlo so that the
share of tokens routing to each expert matches a target.
"""
from __future__ import annotations

import numpy as np

BF16_STD = 0.02


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ------------------------------------------------------------ route shaping

def zipf_share(n_experts: int, top_k: int, s: float = 1.1) -> np.ndarray:
    """Capped Zipf(s) share q_e = min(1, c * rank^-s) with sum q_e = top_k.

    A token picks top_k distinct experts, so no expert can be chosen by more
    than every token; c is found by bisection.
    """
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    lo, hi = 0.0, float(top_k) * 10
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if np.minimum(1.0, c * ranks ** -s).sum() > top_k:
            hi = c
        else:
            lo = c
    return np.minimum(1.0, lo * ranks ** -s)


def hot_share(n_experts: int, top_k: int, hot: int = 8, fraction: float = 0.8) -> np.ndarray:
    """`fraction` of all assignments on `hot` experts, the rest spread evenly."""
    q = np.empty(n_experts)
    q[:hot] = fraction * top_k / hot
    q[hot:] = (1 - fraction) * top_k / (n_experts - hot)
    return np.minimum(q, 1.0)


def route_profile(target: np.ndarray, top_k: int, samples: int = 16384, iters: int = 60,
                  seed: int = 12345) -> np.ndarray:
    """Row-norm multipliers whose Gaussian logits reproduce `target` shares."""
    rng = np.random.default_rng(seed)
    E = target.size
    z = rng.standard_normal((samples, E)).astype(np.float32)
    f = np.ones(E)
    for _ in range(iters):
        logits = z * f[None, :].astype(np.float32)
        top = np.argpartition(-logits, top_k - 1, axis=1)[:, :top_k]
        share = np.bincount(top.ravel(), minlength=E) / samples
        f *= np.clip((np.maximum(target, 1e-4) / np.maximum(share, 1e-4)) ** 0.35, 0.8, 1.25)
        f /= np.exp(np.mean(np.log(f)))
    return f


# --------------------------------------------------------------- host (numpy)

def moe_weights(hidden, inter, experts, shared, seed, router_scale=None, norm=False):
    """BF16 bits of one MoE layer in checkpoint layout, from a numpy stream."""
    rng = np.random.default_rng(seed)
    S = inter * shared

    def normal(shape):
        return f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * BF16_STD)

    router = rng.standard_normal((experts, hidden), dtype=np.float32) * BF16_STD
    if router_scale is not None:
        router *= np.asarray(router_scale, np.float32)[:, None]
    w = {
        "router": f32_to_bf16_bits(router),
        "gate": normal((experts, inter, hidden)),
        "up": normal((experts, inter, hidden)),
        "down": normal((experts, hidden, inter)),
        "shared_gate": normal((S, hidden)),
        "shared_up": normal((S, hidden)),
        "shared_down": normal((hidden, S)),
    }
    if norm:
        w["norm_weight"] = f32_to_bf16_bits(np.ones(hidden, np.float32))
    return w


def int8_overlay(hidden, inter, experts, shared, seed):
    """INT8 block-32 overlay: q uniform in [-127, 127], scales |N(0.002, 0.0005)|."""
    rng = np.random.default_rng(seed)
    S = inter * shared

    def mat(rows, cols, lead=()):
        q = rng.integers(-127, 128, size=lead + (rows, cols), dtype=np.int8)
        s = np.abs(rng.normal(0.002, 0.0005, size=lead + (rows, cols // 32))).astype(np.float32)
        return q, s

    return {
        "gate": mat(inter, hidden, (experts,)),
        "up": mat(inter, hidden, (experts,)),
        "down": mat(hidden, inter, (experts,)),
        "shared_gate": mat(S, hidden),
        "shared_up": mat(S, hidden),
        "shared_down": mat(hidden, S),
    }


def activations(T, hidden, seed):
    return np.random.default_rng(seed).standard_normal((T, hidden), dtype=np.float32)


# ------------------------------------------------------------ device (torch)

def moe_weights_device(hidden, inter, experts, shared, seed, router_scale=None, norm=False,
                       device="cuda"):
    """Same distributions generated on the GPU with torch (bench plumbing)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    S = inter * shared

    def normal(shape):
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * BF16_STD
        return t.to(torch.bfloat16).view(torch.int16)

    router = torch.randn((experts, hidden), generator=g, device=device) * BF16_STD
    if router_scale is not None:
        router *= torch.as_tensor(np.asarray(router_scale, np.float32), device=device)[:, None]
    w = {
        "router": router.to(torch.bfloat16).view(torch.int16),
        "gate": normal((experts, inter, hidden)),
        "up": normal((experts, inter, hidden)),
        "down": normal((experts, hidden, inter)),
        "shared_gate": normal((S, hidden)),
        "shared_up": normal((S, hidden)),
        "shared_down": normal((hidden, S)),
    }
    if norm:
        w["norm_weight"] = torch.ones(hidden, device=device).to(torch.bfloat16).view(torch.int16)
    return w


def int8_overlay_device(hidden, inter, experts, shared, seed, device="cuda"):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    S = inter * shared

    def mat(shape):
        q = torch.randint(-127, 128, shape, generator=g, device=device, dtype=torch.int8)
        s_shape = shape[:-1] + (shape[-1] // 32,)
        s = (torch.randn(s_shape, generator=g, device=device) * 0.0005 + 0.002).abs()
        return q, s

    return {
        "gate": mat((experts, inter, hidden)),
        "up": mat((experts, inter, hidden)),
        "down": mat((experts, hidden, inter)),
        "shared_gate": mat((S, hidden)),
        "shared_up": mat((S, hidden)),
        "shared_down": mat((hidden, S)),
    }
