"""Pins for oracle/sampling.py: library argmax, reductions to greedy, kept-set form."""
import numpy as np
import torch

from oracle import sampling as S


def test_greedy_is_first_max_index():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, -1.0, 0.0, 0.0]])
    assert S.greedy(logits).tolist() == [1, 0]


def test_top_k_one_and_tiny_top_p_reduce_to_argmax():
    g = torch.Generator().manual_seed(0)
    for _ in range(5):
        row = torch.randn(1000, generator=g)
        best = int(row.argmax())
        assert np.flatnonzero(S.kept_set(row, 0.7, 1, 1.0)).tolist() == [best]
        assert np.flatnonzero(S.kept_set(row, 1.3, 0, 1e-9)).tolist() == [best]
        noise = np.random.default_rng(1).exponential(size=1000)
        assert S.sample_with_noise(row, 0.7, 1, 1.0, noise) == best


def test_top_p_kept_set_is_the_crossing_prefix():
    row = torch.log(torch.tensor([0.1, 0.4, 0.2, 0.3], dtype=torch.float64))
    # Sorted: 0.4 (1), 0.3 (3), 0.2 (2), 0.1 (0); prefix masses before: 0, .4, .7, .9
    assert np.flatnonzero(S.kept_set(row, 1.0, 0, 0.5)).tolist() == [1, 3]
    assert np.flatnonzero(S.kept_set(row, 1.0, 0, 0.35)).tolist() == [1]
    assert np.flatnonzero(S.kept_set(row, 1.0, 0, 0.75)).tolist() == [1, 2, 3]
    assert S.kept_set(row, 1.0, 0, 1.0).all()
    # top-k first, then top-p renormalised over the candidates.
    assert np.flatnonzero(S.kept_set(row, 1.0, 2, 0.6)).tolist() == [1, 3]
    assert np.flatnonzero(S.kept_set(row, 1.0, 2, 0.5)).tolist() == [1]


def test_ties_follow_stable_index_order():
    row = torch.tensor([1.0, 2.0, 2.0, 2.0, 0.0])
    assert np.flatnonzero(S.kept_set(row, 1.0, 2, 1.0)).tolist() == [1, 2]
    # Equal masses 1/3 each among the three 2.0 tokens (plus small others).
    row = torch.tensor([2.0, 2.0, 2.0])
    assert np.flatnonzero(S.kept_set(row, 1.0, 0, 0.5)).tolist() == [0, 1]


def test_sampling_frequencies_follow_softmax():
    row = torch.log(torch.tensor([0.5, 0.3, 0.2]))
    rng = np.random.default_rng(3)
    counts = np.zeros(3)
    for _ in range(4000):
        counts[S.sample_with_noise(row, 1.0, 0, 1.0, rng.exponential(size=3))] += 1
    assert np.allclose(counts / 4000, [0.5, 0.3, 0.2], atol=0.03)
