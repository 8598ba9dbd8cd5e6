"""ImportanceScorer.get_tier_assignments and get_aggregated_scores
(akv/importance.py:174-243) on host score tensors (tier bookkeeping, no kernels):
the tiers partition the positions, hold hot_budget / warm_budget / the rest, are
ascending, every hot score is >= every warm score >= every cold score (protected
positions counting as +inf), and equal scores rank the lower index as less
important, as get_eviction_candidates does."""
import itertools

import numpy as np
import pytest
import torch


def _scorer(scores, protect_start=2, protect_end=2):
    from akv.importance import ImportanceConfig, ImportanceScorer
    sc = ImportanceScorer(ImportanceConfig(initial_tokens_protected=protect_start,
                                           recent_tokens_protected=protect_end))
    sc._scores[0] = torch.tensor(scores, dtype=torch.float32)
    return sc


@pytest.mark.parametrize("seed", range(6))
def test_tiers_partition_and_order(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    scores = rng.integers(0, 6, n).astype(np.float32)  # many ties
    ps, pe = int(rng.integers(0, 4)), int(rng.integers(0, 4))
    sc = _scorer(scores.tolist() + [9.0] * 3, ps, pe)  # stored scores may run past seq_len
    for hb, wb in itertools.product((0, 1, 5, 50), (0, 3, 50)):
        hot, warm, cold = sc.get_tier_assignments(0, n, hb, wb)
        assert hot.numel() == min(hb, n) and warm.numel() == min(hb + wb, n) - min(hb, n)
        allpos = torch.cat([hot, warm, cold]).sort().values
        assert torch.equal(allpos, torch.arange(n))
        for t in (hot, warm, cold):
            assert (t[1:] > t[:-1]).all()
        eff = scores.copy()
        eff[:min(ps, n)] = np.inf
        if pe:
            eff[max(0, n - pe):] = np.inf
        # rank key: (effective score, index); hotter tiers hold the larger keys
        key = lambda i: (eff[i], i)
        for hi, lo in ((hot, warm), (warm, cold), (hot, cold)):
            if hi.numel() and lo.numel():
                assert min(key(i) for i in hi.tolist()) > max(key(i) for i in lo.tolist())


def test_reference_case_protected_and_important_are_hot():
    s = [0.1] * 20
    s[5], s[6] = 0.9, 0.8
    hot, warm, cold = _scorer(s).get_tier_assignments(0, seq_len=20, hot_budget=8, warm_budget=6)
    assert (hot.numel(), warm.numel(), cold.numel()) == (8, 6, 6)
    assert {0, 1, 18, 19, 5, 6} <= set(hot.tolist())


def test_no_scores_splits_by_position():
    from akv.importance import ImportanceScorer
    hot, warm, cold = ImportanceScorer().get_tier_assignments(3, seq_len=10, hot_budget=4, warm_budget=3)
    assert hot.tolist() == [0, 1, 2, 3] and warm.tolist() == [4, 5, 6] and cold.tolist() == [7, 8, 9]


def test_aggregated_scores_pad_and_average():
    from akv.importance import ImportanceScorer
    sc = ImportanceScorer()
    assert sc.get_aggregated_scores() is None
    sc._scores[0] = torch.tensor([1.0, 2.0, 3.0])
    sc._scores[4] = torch.tensor([3.0, 4.0, 5.0, 6.0, 7.0])
    np.testing.assert_array_equal(sc.get_aggregated_scores().numpy(), [2.0, 3.0, 4.0, 3.0, 3.5])
