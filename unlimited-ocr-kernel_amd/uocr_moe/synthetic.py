"""Seeded synthetic MoE-layer workloads (no checkpoints are available offline).

Weights follow the benchmark definitions: BF16 N(0, 0.02) rounded to nearest
even; INT8 overlay int8 uniform in [-127, 127] with per-32-block scales
|N(0.002, 0.0005)|; activations N(0, 1). The router has no bias
(src/decoder/mod.rs:126 passes bias None), so expert popularity is shaped
through the router rows:

* `route_profile` scales router rows (a larger row norm gives an expert
  larger logits more often), calibrated by Monte Carlo to target shares.
  With zero-mean inputs every logit is symmetric, so an expert is chosen by
  at most half of the tokens: targets are capped below that (`zipf_share`'s
  cap). Scaling past it only makes the other experts' softmax probabilities
  underflow to exact zeros, which moe::route then breaks by lowest id.
* `hot_tilt` reaches shares above one half: the hot experts' router rows
  are tilted toward a unit direction d and the input carries a small mean
  mu * d (|mu d| = 4 against |z| = sqrt(H) for z ~ N(0, 1)), so the hot
  logits have a positive mean. The tilts are calibrated for the effective
  mean a layer of the residual stack sees after RMSNorm.
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

ZIPF_CAP = 0.45


def zipf_share(n_experts: int, top_k: int, s: float = 1.1, cap: float = ZIPF_CAP) -> np.ndarray:
    """Capped Zipf(s) share q_e = min(cap, c * rank^-s) with sum q_e = top_k.

    q_e is the fraction of tokens that choose expert e. A token picks top_k
    distinct experts, and with zero-mean N(0, 1) inputs (as the 1024-token
    prefill specifies) a router row can win at most half of the tokens, so
    the head of the distribution is capped just below that; c is found by
    bisection.
    """
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    lo, hi = 0.0, float(top_k) * 10
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if np.minimum(cap, c * ranks ** -s).sum() > top_k:
            hi = c
        else:
            lo = c
    return np.minimum(cap, lo * ranks ** -s)


def hot_share(n_experts: int, top_k: int, hot: int = 8, fraction: float = 0.8) -> np.ndarray:
    """`fraction` of all assignments on `hot` experts, the rest spread evenly."""
    q = np.empty(n_experts)
    q[:hot] = fraction * top_k / hot
    q[hot:] = (1 - fraction) * top_k / (n_experts - hot)
    return np.minimum(q, 1.0)


def route_profile(target: np.ndarray, top_k: int, samples: int = 16384, iters: int = 60,
                  seed: int = 12345, max_ratio: float = 30.0) -> np.ndarray:
    """Row-norm multipliers whose Gaussian logits reproduce `target` shares
    (each at most one half). The multipliers stay within a factor
    `max_ratio` of their geometric mean, so softmax probabilities never
    underflow to ties."""
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
        f = np.clip(f, 1.0 / max_ratio, max_ratio)
    return f


# Input mean of the hot-expert workload along the tilt direction, and the
# growth of the residual stream's mean square per layer of the 12-layer
# stack (each layer adds a nearly independent output of rms 0.256 to rows of
# rms 1), which dilutes the normalised mean the deeper layers see.
HOT_MEAN = 4.0
STACK_GROWTH = 0.0655


def tilt_direction(hidden: int, seed: int = 4242) -> np.ndarray:
    """The unit direction d of the hot-expert tilt (float32)."""
    d = np.random.default_rng(seed).standard_normal(hidden)
    return (d / np.linalg.norm(d)).astype(np.float32)


def hot_tilt(target: np.ndarray, top_k: int, hidden: int, layer: int = 0,
             mean: float = HOT_MEAN, samples: int = 16384, iters: int = 80,
             seed: int = 7) -> np.ndarray:
    """Tilts beta_e (router row e gets beta_e * d added before the 0.02
    scale) so that layer `layer` of the stack routes `target` shares.

    Model: after RMSNorm a row is z + m d with z ~ N(0, 1) and
    m = mean / sqrt(1 + layer * STACK_GROWTH); logit_e / 0.02 =
    g_e . z + beta_e (m + d . z), with g_e . z ~ N(0, hidden) independent
    per expert and d . z ~ N(0, 1) shared. Monte Carlo, additive updates."""
    rng = np.random.default_rng(seed)
    E = target.size
    m = mean / np.sqrt(1.0 + layer * STACK_GROWTH)
    n = rng.standard_normal((samples, E)) * np.sqrt(hidden)
    w = rng.standard_normal((samples, 1))
    beta = np.zeros(E)
    for _ in range(iters):
        logits = n + beta[None, :] * (m + w)
        top = np.argpartition(-logits, top_k - 1, axis=1)[:, :top_k]
        share = np.bincount(top.ravel(), minlength=E) / samples
        beta += 8.0 * (target - share)
    return beta


# --------------------------------------------------------------- host (numpy)

def moe_weights(hidden, inter, experts, shared, seed, router_scale=None, norm=False,
                router_tilt=None):
    """BF16 bits of one MoE layer in checkpoint layout, from a numpy stream.
    router_tilt: (beta [E], d [hidden]) adds beta_e * d to router row e
    before the 0.02 scale."""
    rng = np.random.default_rng(seed)
    S = inter * shared

    def normal(shape):
        return f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * BF16_STD)

    router = rng.standard_normal((experts, hidden), dtype=np.float32)
    if router_tilt is not None:
        beta, d = router_tilt
        router += np.asarray(beta, np.float32)[:, None] * np.asarray(d, np.float32)[None, :]
    router *= BF16_STD
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
                       device="cuda", router_tilt=None):
    """Same distributions generated on the GPU with torch (bench plumbing)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    S = inter * shared

    def normal(shape):
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * BF16_STD
        return t.to(torch.bfloat16).view(torch.int16)

    router = torch.randn((experts, hidden), generator=g, device=device)
    if router_tilt is not None:
        beta, d = router_tilt
        router += (torch.as_tensor(np.asarray(beta, np.float32), device=device)[:, None]
                   * torch.as_tensor(np.asarray(d, np.float32), device=device)[None, :])
    router *= BF16_STD
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


def hot_stack_layer_device(hidden, inter, experts, shared, top_k, layer, hot=8, fraction=0.8,
                           seed_base=1000, device="cuda"):
    """Layer `layer` of the hot-expert stack: BF16 weights from the seeded
    stream seed_base + layer, the router tilted so that `fraction` of the
    assignments reach the first `hot` experts at that depth, norm weight
    ones."""
    beta = hot_tilt(hot_share(experts, top_k, hot, fraction), top_k, hidden, layer)
    return moe_weights_device(hidden, inter, experts, shared, seed=seed_base + layer, norm=True,
                              device=device, router_tilt=(beta, tilt_direction(hidden)))


def hot_stack_input_device(T, hidden, seed=1, device="cuda"):
    """The hot-expert stack's input: N(0, 1) rows plus HOT_MEAN * d."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    x = torch.randn((T, hidden), generator=g, device=device)
    d = torch.as_tensor(tilt_direction(hidden), device=device)
    return x + HOT_MEAN * d[None, :]
