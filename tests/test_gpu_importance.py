"""Importance on the device: the observation-window sum + average pooling of
akv_importance_update and every ImportanceScorer strategy against the oracle
(akv/importance.py:73-164)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev
from oracle import importance as oimp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,W,ks", [(10, 700, 4, 7), (3, 300, 8, 5), (6, 12, 6, 4), (5, 6, 2, 7), (1, 513, 32, 7),
                                      (40, 1000, 32, 64)])
def test_observation_window_pooling(M, N, W, ks):
    from akv.importance import accumulate
    announce(f"importance window M{M} N{N} W{W} ks{ks}")
    rng = np.random.default_rng(M * 1000 + N)
    a = rng.random((2, 3, M, N)).astype(np.float32)
    a /= a.sum(-1, keepdims=True)
    s0 = rng.random(N).astype(np.float32)
    sc = to_dev(s0)
    accumulate(sc, to_dev(a), 0.9, q_window=W, pool_kernel=ks)
    exp = oimp.scorer_update(s0, a, "observation_window", 0.9, observation_window=W, pooling_kernel=ks)
    np.testing.assert_allclose(sc.cpu().numpy(), exp, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("strategy", ["attention_accumulation", "importance", "observation_window", "heavy_hitter",
                                      "recency_weighted", "hybrid", "fifo"])
def test_scorer_strategies_three_steps(strategy):
    from akv.importance import ImportanceConfig, ImportanceScorer, ScoringStrategy
    announce(f"ImportanceScorer {strategy}")
    cfg = ImportanceConfig(strategy=ScoringStrategy(strategy), decay_factor=0.8, observation_window=3,
                           pooling_kernel=5)
    sc = ImportanceScorer(cfg)
    ref = None
    rng = np.random.default_rng(len(strategy))
    for step, (M, N) in enumerate(((6, 40), (1, 41), (1, 42))):
        a = rng.random((2, 4, M, N)).astype(np.float32)
        a /= a.sum(-1, keepdims=True)
        sc.update(to_dev(a), layer_idx=3)
        ref = oimp.scorer_update(ref, a, strategy, 0.8, observation_window=3, pooling_kernel=5,
                                 attention_weight=cfg.attention_weight, recency_weight=cfg.recency_weight)
        np.testing.assert_allclose(sc.get_scores(3).cpu().numpy(), ref, rtol=2e-5, atol=1e-6, err_msg=f"step {step}")
    assert sc.step_count == 3 and sc.stats()["total_seq_len"] == 42


def test_default_scorer_is_hybrid_and_updates():
    from akv.importance import ImportanceScorer
    announce("ImportanceScorer default config")
    sc = ImportanceScorer()
    a = torch.softmax(torch.randn(1, 2, 1, 16, device="cuda"), -1)
    sc.update(a, 0)
    s = sc.get_scores(0)
    assert s.shape == (16,) and torch.isfinite(s).all()
    assert float(s.max()) <= 0.7 + 0.3 + 1e-6  # normalised EMA (<= 0.7) plus recency (<= 0.3)


def test_aggregated_scores_and_tiers_on_device():
    """After device updates of two layers: the aggregate is the layers' mean on the device,
    and the tier split of a layer is taken on its scores' device."""
    from akv.importance import ImportanceConfig, ImportanceScorer, ScoringStrategy
    announce("ImportanceScorer aggregate / tiers on the device")
    sc = ImportanceScorer(ImportanceConfig(strategy=ScoringStrategy.ATTENTION_ACCUMULATION,
                                           initial_tokens_protected=2, recent_tokens_protected=2))
    rng = np.random.default_rng(3)
    a = rng.random((1, 2, 1, 16)).astype(np.float32)
    a /= a.sum(-1, keepdims=True)
    sc.update(to_dev(a), layer_idx=0)
    sc.update(to_dev(a * 0.5), layer_idx=1)
    agg = sc.get_aggregated_scores()
    assert agg.is_cuda and agg.shape == (16,)
    torch.testing.assert_close(agg, (sc.get_scores(0) + sc.get_scores(1)) / 2)
    hot, warm, cold = sc.get_tier_assignments(0, 16, 6, 4)
    assert hot.is_cuda and (hot.numel(), warm.numel(), cold.numel()) == (6, 4, 6)
    assert {0, 1, 14, 15} <= set(hot.tolist())
