"""The routing/dispatch checker the GPU parity tests and bench.py use
(oracle/routing_check.py), pinned on the CPU: its expected dispatch equals
the oracle's own (src/decoder/mod.rs:127-141) on random routings, a tie flip
within 1e-6 is accepted with the dispatch still checked, and planted
mistakes (a reordered permutation, a flip outside the tie window, a wrong
carried weight, a different order outside the tie set) are rejected."""
import numpy as np
import pytest

import oracle as orc
import routing_check as rc


def _oracle_trace(T, E, K, seed):
    """The oracle's routing and dispatch of random logits (orc_moe_experts
    on a tiny layer whose router rows are the identity, so the logits are
    the input)."""
    rng = np.random.default_rng(seed)
    H = E
    router = orc.f32_to_bf16(np.eye(E, H, dtype=np.float32))
    z = lambda *s: np.zeros(s, np.uint16)
    w = orc.MoeWeights(hidden=H, inter=32, n_experts=E, top_k=K, n_shared=1, normalize=True,
                       router=router, gate=z(E, 32, H), up=z(E, 32, H), down=z(E, H, 32),
                       shared_gate=z(32, H), shared_up=z(32, H), shared_down=z(H, 32))
    x = (rng.standard_normal((T, H)) * 2).astype(np.float32)
    _, tr = orc.moe_experts(w, x, trace=True)
    return tr


def _as_gpu(tr):
    return {"topk_ids": tr.topk_ids.copy(), "topk_weights": tr.topk_weights.copy(),
            "expert_offsets": tr.expert_offsets.copy(), "perm_rows": tr.perm_rows.copy(),
            "perm_weights": tr.perm_weights.copy()}


@pytest.mark.parametrize("T,E,K,seed", [(1, 8, 2, 0), (37, 16, 4, 1), (300, 64, 6, 2)])
def test_expected_dispatch_is_the_oracles(T, E, K, seed):
    tr = _oracle_trace(T, E, K, seed)
    off, perm = rc.expected_dispatch(tr.topk_ids, E)
    assert np.array_equal(off, tr.expert_offsets)
    assert np.array_equal(perm, tr.perm_rows)
    rc.check_dispatch(_as_gpu(tr), tr, [], E)


def test_tie_flip_keeps_the_dispatch_checked():
    T, E, K = 40, 16, 4
    tr = _oracle_trace(T, E, K, 3)
    g = _as_gpu(tr)
    t = 5
    order = np.argsort(-tr.logits[t], kind="stable")
    kth, nxt = order[K - 1], order[K]
    # Make the k-th and (k+1)-th logits of token t tie within 1e-6 in the
    # oracle's view, and let the "GPU" pick the other one.
    tr.logits[t, nxt] = tr.logits[t, kth] - np.float32(5e-7)
    ids = g["topk_ids"][t].copy()
    ids[ids == kth] = nxt
    g["topk_ids"][t] = ids
    off, perm = rc.expected_dispatch(g["topk_ids"], E)
    g["expert_offsets"], g["perm_rows"] = off.astype(np.int32), perm.astype(np.int32)
    expert_of = np.repeat(np.arange(E), np.diff(off))
    slot = np.argmax(g["topk_ids"][perm] == expert_of[:, None], axis=1)
    g["perm_weights"] = g["topk_weights"][perm, slot]
    ties = rc.tie_tokens(tr.topk_ids, tr.logits, g["topk_ids"], K)
    assert ties == [t]
    rc.check_dispatch(g, tr, ties, E)
    # The same flip with the tie window missed is rejected.
    tr.logits[t, nxt] = tr.logits[t, kth] - np.float32(1e-3)
    with pytest.raises(rc.RoutingMismatch):
        rc.tie_tokens(tr.topk_ids, tr.logits, g["topk_ids"], K)
    # ... unless a stated input perturbation bound covers it.
    slack = np.zeros(T)
    slack[t] = 2e-3
    assert rc.tie_tokens(tr.topk_ids, tr.logits, g["topk_ids"], K, slack=slack) == [t]


def test_planted_dispatch_mistakes_are_rejected():
    T, E, K = 64, 16, 4
    tr = _oracle_trace(T, E, K, 4)
    # Two rows of one expert swapped.
    g = _as_gpu(tr)
    e = int(np.argmax(np.diff(tr.expert_offsets)))
    p = tr.expert_offsets[e]
    g["perm_rows"][p], g["perm_rows"][p + 1] = g["perm_rows"][p + 1], g["perm_rows"][p]
    with pytest.raises(rc.RoutingMismatch):
        rc.check_dispatch(g, tr, [], E)
    # A carried weight that is not the token's routing weight.
    g = _as_gpu(tr)
    g["perm_weights"][3] = np.nextafter(g["perm_weights"][3], np.float32(2))
    with pytest.raises(rc.RoutingMismatch):
        rc.check_dispatch(g, tr, [], E)
    # Offsets that disagree with the ids.
    g = _as_gpu(tr)
    g["expert_offsets"][1] += 1
    with pytest.raises(rc.RoutingMismatch):
        rc.check_dispatch(g, tr, [], E)
    # A GPU self-consistent with its ids that differ from the oracle's on a
    # token the tie set does not name.
    g = _as_gpu(tr)
    t = 9
    order = np.argsort(-tr.logits[t], kind="stable")
    ids = g["topk_ids"][t].copy()
    ids[ids == order[K - 1]] = order[K]
    g["topk_ids"][t] = ids
    off, perm = rc.expected_dispatch(g["topk_ids"], E)
    g["expert_offsets"], g["perm_rows"] = off, perm
    g.pop("perm_weights")
    with pytest.raises(rc.RoutingMismatch):
        rc.check_dispatch(g, tr, [], E)
    rc.check_dispatch(g, tr, [t], E)  # named as a tie it passes


def test_logit_slack_bounds_the_logit_change():
    rng = np.random.default_rng(6)
    r = rng.standard_normal((8, 32)) * 0.02
    a = rng.standard_normal((5, 32))
    b = a + rng.standard_normal((5, 32)) * 1e-4
    s = rc.logit_slack(a, b, r)
    la, lb = a @ r.T, b @ r.T
    # Any difference of two logits moves by at most the slack.
    for t in range(5):
        d = (la[t][:, None] - la[t][None, :]) - (lb[t][:, None] - lb[t][None, :])
        assert np.abs(d).max() <= s[t] + 1e-15
