"""Synthetic workload generators (CPU): the stated distributions of the C3, C4, C5 inputs."""
import numpy as np
import torch

from kvq.synth import ar1, c4_inputs, gen


def test_ar1_stationary_and_correlated():
    x = ar1((3, 40000), 0.95, gen("cpu", 0), "cpu").double().numpy()
    assert abs(x.std() - 1.0) < 0.05
    for row in x:
        assert abs(np.corrcoef(row[:-1], row[1:])[0, 1] - 0.95) < 0.01


def test_ar1_obeys_recursion():
    # the chunked closed form equals the sequential recursion on the same innovations
    g = gen("cpu", 3)
    x = ar1((2, 1000), 0.9, g, "cpu", chunk=64).double()
    g2 = gen("cpu", 3)
    e = torch.randn((2, 1000), generator=g2).double() * np.sqrt(1 - 0.81)
    prev = torch.randn((2,), generator=g2).double()
    ref = torch.empty_like(e)
    for t in range(1000):
        prev = 0.9 * prev + e[:, t]
        ref[:, t] = prev
    assert float((x - ref).abs().max()) < 1e-4


def test_c4_heavy_hitters():
    q, K, V = c4_inputs("cpu", T=2000, B=1, steps=2)
    assert q.shape == (2, 1, 32, 1, 128) and K.shape == (1, 8, 2000, 128)
    hot = (K.float().mean(-1) > 1.5).sum(-1)
    assert (hot == 20).all()
