"""Device policy sampling (cg_masked_probabilities, cg_sample_rows) against the oracle's
restatement of cardgym/rl/ppo.py:75-94.

Bars: sample_rows is exact (same probabilities and uniforms give the same indices,
including uniforms placed exactly on and next to every float32 running sum); the
probabilities agree to 8 float32 ulps and 1 ulp on average: max, masking, the pairwise
normaliser and the division are the same operations in the same order, but the device exp
and numpy's exp are different implementations (up to ~2 ulps each), and a weight's
difference reaches its probability both directly and through the normaliser."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from card_playing_gym_amd.rl import masked_probabilities, sample_rows
from oracle import sampling as ref

pytestmark = pytest.mark.gpu


def case(rows: int, width: int, seed: int, density: float = 0.4):
    rng = np.random.default_rng(seed)
    mask = rng.random((rows, width)) < density
    mask[np.arange(rows), rng.integers(0, width, rows)] = True
    logits = (rng.normal(size=(rows, width)) * 3).astype(np.float32)
    return logits, mask, rng


@pytest.mark.parametrize("rows, width", [(1, 1), (200, 9), (33, 129), (4096, 512), (64, 1000)])
def test_masked_probabilities_match_the_oracle(device, rows, width):
    logits, mask, _ = case(rows, width, rows + width)
    got = masked_probabilities(torch.from_numpy(logits).to(device), torch.from_numpy(mask).to(device)).cpu().numpy()
    want = ref.masked_probabilities(logits, mask)
    assert (got[~mask] == 0).all()
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 8, ulps.max()
    assert ulps[mask].mean() <= 1.0, ulps[mask].mean()
    np.testing.assert_allclose(got.sum(1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("rows, width", [(200, 9), (4096, 512), (64, 1000)])
def test_sample_rows_is_exact_at_every_boundary(device, rows, width):
    logits, mask, rng = case(rows, width, 7 + width)
    probs = ref.masked_probabilities(logits, mask)
    cdf = np.cumsum(probs, axis=1).astype(np.float64)
    cols = rng.integers(0, width, rows)
    on = cdf[np.arange(rows), cols]
    trials = [rng.random(rows), np.zeros(rows), np.ones(rows), on, np.nextafter(on, 2.0), np.nextafter(on, -1.0)]
    p_dev, m_dev = torch.from_numpy(probs).to(device), torch.from_numpy(mask).to(device)
    for uniforms in trials:
        got = sample_rows(p_dev, m_dev, torch.from_numpy(uniforms).to(device)).cpu().numpy()
        want = ref.sample_rows(probs, mask, uniforms)
        assert (got == want).all()
        assert mask[np.arange(rows), got].all()


def test_device_probabilities_then_sampling(device):
    """The composed device path equals the reference's sampling of the device's own
    probabilities, so only the exp's last bit can move a pick, never the sampling."""

    logits, mask, rng = case(4096, 512, 11)
    m_dev = torch.from_numpy(mask).to(device)
    probs = masked_probabilities(torch.from_numpy(logits).to(device), m_dev)
    uniforms = rng.random(4096)
    got = sample_rows(probs, m_dev, torch.from_numpy(uniforms).to(device)).cpu().numpy()
    assert (got == ref.sample_rows(probs.cpu().numpy(), mask, uniforms)).all()


def test_rows_without_a_legal_entry_follow_numpy(device):
    logits = np.zeros((2, 5), dtype=np.float32)
    mask = np.array([[False] * 5, [False, True, False, False, False]])
    with np.errstate(invalid="ignore"):
        want = ref.masked_probabilities(logits, mask)
    got = masked_probabilities(torch.from_numpy(logits).to(device), torch.from_numpy(mask).to(device)).cpu().numpy()
    assert np.isnan(got[0]).all() and np.isnan(want[0]).all()
    assert (got[1] == want[1]).all()
    uniforms = np.array([0.5, 0.5])
    assert (sample_rows(torch.from_numpy(got).to(device), torch.from_numpy(mask).to(device),
                        torch.from_numpy(uniforms).to(device)).cpu().numpy() == ref.sample_rows(want, mask, uniforms)).all()
