"""Synthetic k-quant generators (engine_amd/synth.py) on the CPU: the torch
generator's BASELINE distribution, and the centered variant the random-weight
decoder benchmark uses, decoded by the oracle."""
import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

torch = pytest.importorskip("torch")


def _weights(t, centered, seed=1):
    g = torch.Generator()
    g.manual_seed(seed)
    enc = synth.kquant_torch(t, 1024, 64, g, torch.device("cpu"), centered=centered).numpy()
    assert enc.size == 4 * 64 * synth.BLOCK_BYTES[t]
    return enc, np.asarray(O.dequantize_tensor(t, enc), np.float64)


@pytest.mark.parametrize("t", (12, 13))
def test_baseline_distribution_shares_a_positive_mean(t):
    enc, w = _weights(t, False)
    blocks = enc.reshape(-1, synth.BLOCK_BYTES[t])
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)
    assert 0.001 <= d.min() and d.max() <= 0.02 and 0.001 <= dmin.min() and dmin.max() <= 0.02
    assert w.mean() / w.std() > 0.5


@pytest.mark.parametrize("t,mean_q", ((12, 7.5), (13, 15.5)))
def test_centered_weights_have_zero_mean(t, mean_q):
    enc, w = _weights(t, True)
    blocks = enc.reshape(-1, synth.BLOCK_BYTES[t])
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(dmin, (d * mean_q).astype(np.float16).astype(np.float32))
    assert abs(w.mean() / w.std()) < 0.05


def test_q6k_is_centered_either_way():
    for c in (False, True):
        _, w = _weights(14, c)
        assert abs(w.mean() / w.std()) < 0.05
