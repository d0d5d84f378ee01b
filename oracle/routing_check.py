"""Routing and dispatch checks of a GPU forward against the oracle.

TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's post-timing parity
check; the product library never calls it.

The bar (the path's routing parity rule): a token's top-k expert set equals
the oracle's except where the oracle's logits tie within 1e-6, i.e. every
expert in the symmetric difference has a logit within 1e-6 of the oracle's
k-th largest (`moe::route`, src/decoder/moe.rs:7-30: probability
descending, id ascending). The dispatch is the reference's assignment order
(src/decoder/mod.rs:127-141): for each expert in ascending id, the rows that
chose it in ascending row order. Ties do not remove the dispatch check: the
GPU's permutation must be exactly the stable order of its own top-k ids, and
on every token outside the tie set it must equal the oracle's.
"""
from __future__ import annotations

import numpy as np

TIE = 1e-6


class RoutingMismatch(AssertionError):
    pass


def _kth(logits_row: np.ndarray, k: int) -> float:
    return float(np.sort(logits_row)[::-1][k - 1])


def tie_tokens(ref_ids, ref_logits, gpu_ids, k, tie=TIE, slack=None):
    """Tokens whose selected set differs from the oracle's. Raises unless
    every differing expert's oracle logit lies within `tie` (+ slack[t], a
    per-token bound on how far the logits can move, when given) of the
    oracle's k-th largest logit."""
    ref_ids = np.asarray(ref_ids)
    gpu_ids = np.asarray(gpu_ids)
    bad = []
    for t in range(ref_ids.shape[0]):
        a, b = set(ref_ids[t].tolist()), set(gpu_ids[t].tolist())
        if a == b:
            continue
        kth = _kth(ref_logits[t], k)
        lim = tie + (0.0 if slack is None else float(slack[t]))
        for e in sorted(a ^ b):
            gap = abs(float(ref_logits[t][e]) - kth)
            if gap > lim:
                raise RoutingMismatch(f"token {t}: expert {e} differs with logit gap {gap:.3e} "
                                      f"to the k-th (allowed {lim:.3e})")
        bad.append(t)
    return bad


def expected_dispatch(ids, n_experts):
    """(expert_offsets [E+1], perm_rows [T*k]) of the reference's assignment
    order for the top-k ids [T, k]: experts ascending, rows ascending."""
    ids = np.asarray(ids)
    counts = np.bincount(ids.ravel(), minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    perm = [np.nonzero((ids == e).any(axis=1))[0] for e in range(n_experts)]
    return offsets, np.concatenate(perm).astype(np.int64) if perm else np.zeros(0, np.int64)


def check_dispatch(gpu, ref, ties, n_experts):
    """The GPU trace's dispatch (expert_offsets, perm_rows and, when present,
    perm_weights) against the stable order of its own top-k ids, exactly;
    and against the oracle's trace on every token outside `ties`."""
    ids = np.asarray(gpu["topk_ids"])
    off, perm = expected_dispatch(ids, n_experts)
    g_off = np.asarray(gpu["expert_offsets"]).astype(np.int64)
    g_perm = np.asarray(gpu["perm_rows"]).astype(np.int64)
    if not np.array_equal(g_off, off):
        raise RoutingMismatch("expert offsets differ from the GPU's own top-k ids")
    if not np.array_equal(g_perm, perm):
        raise RoutingMismatch("permutation differs from the stable order of the GPU's own ids")
    if "perm_weights" in gpu and "topk_weights" in gpu:
        w = np.asarray(gpu["topk_weights"])
        expert_of = np.repeat(np.arange(n_experts), np.diff(off))
        slot = np.argmax(ids[perm] == expert_of[:, None], axis=1)
        want = w[perm, slot]
        if not np.array_equal(np.asarray(gpu["perm_weights"]).view(np.uint32),
                              np.ascontiguousarray(want).view(np.uint32)):
            raise RoutingMismatch("permuted weights are not the routing weights they carry")
    # Outside the tie set the order equals the oracle's, position by position
    # among the remaining tokens of each expert.
    r_off = np.asarray(ref.expert_offsets).astype(np.int64)
    r_perm = np.asarray(ref.perm_rows).astype(np.int64)
    tie_mask = np.zeros(ids.shape[0], bool)
    tie_mask[list(ties)] = True
    g_lab = np.repeat(np.arange(n_experts), np.diff(off))
    r_lab = np.repeat(np.arange(n_experts), np.diff(r_off))
    gk, rk = ~tie_mask[g_perm], ~tie_mask[r_perm]
    if not (np.array_equal(g_lab[gk], r_lab[rk]) and np.array_equal(g_perm[gk], r_perm[rk])):
        raise RoutingMismatch("dispatch differs from the oracle's outside the tie set")
    if not ties and not (np.array_equal(g_off, r_off) and np.array_equal(g_perm, r_perm)):
        raise RoutingMismatch("dispatch differs from the oracle's with no tie")


def logit_slack(xn_a, xn_b, router_f32):
    """Per-row bound on how far any logit difference (between two experts)
    can move when the normalised input changes from xn_b to xn_a: twice
    max_e sum_k |xa_k - xb_k| |r_ek|, in float64."""
    d = np.abs(np.asarray(xn_a, np.float64) - np.asarray(xn_b, np.float64))
    return 2.0 * (d @ np.abs(np.asarray(router_f32, np.float64)).T).max(axis=1)
