"""Temperature / top-k / top-p sampling (mini_vllm/sampler.py) on the CPU, against the
numpy oracle (oracle/sampler.py), and the oracle pinned by closed forms: the
properties the reference's own sampler tests check (tests/test_sampler.py), here
asserted of the restatement and of the library alike."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_vllm.sampler import SamplingParams, sample, sampling_probabilities
from oracle import sampler as osm

VOCAB = 64


def _logits(rows=4, vocab=VOCAB, seed=0):
    return torch.randn(rows, vocab, generator=torch.Generator().manual_seed(seed))


def _oracle(logits, params: SamplingParams):
    return osm.sampling_probabilities(logits.float().numpy(), params.temperature, params.top_k,
                                      params.top_p)


# ----------------------------------------------------------- oracle pins


def test_oracle_temperature_one_is_the_softmax():
    x = _logits().numpy().astype(np.float64)
    want = np.exp(x - x.max(1, keepdims=True))
    want /= want.sum(1, keepdims=True)
    assert np.allclose(osm.sampling_probabilities(x, 1.0, 0, 1.0), want, rtol=0, atol=1e-15)


@pytest.mark.parametrize("k", [1, 2, 5, 40])
def test_oracle_top_k_keeps_the_k_largest_logits(k):
    x = _logits().numpy()
    kept = osm.sampling_probabilities(x, 1.0, k, 1.0) > 0
    expect = np.zeros_like(kept)
    np.put_along_axis(expect, np.argsort(-x, axis=1)[:, :k], True, axis=1)
    assert np.array_equal(kept, expect)


def test_oracle_top_p_nucleus_is_the_shortest_prefix_reaching_p():
    x = _logits(8).numpy()
    full = osm.sampling_probabilities(x, 1.0, 0, 1.0)
    kept = osm.sampling_probabilities(x, 1.0, 0, 0.9) > 0
    for row in range(8):
        masses = np.sort(full[row][kept[row]])[::-1]
        assert masses.sum() >= 0.9 and masses[:-1].sum() < 0.9


def test_oracle_uniform_rows_keep_the_token_that_crosses_p():
    x = np.zeros((1, 4))
    assert (osm.sampling_probabilities(x, 1.0, 0, 0.5) > 0).sum() == 2
    assert (osm.sampling_probabilities(x, 1.0, 0, 0.6) > 0).sum() == 3
    # ties keep vocabulary order: the first two token ids
    assert np.array_equal(osm.sampling_probabilities(x, 1.0, 0, 0.5)[0] > 0, [1, 1, 0, 0])


def test_oracle_top_k_one_is_greedy_and_greedy_is_one_hot():
    x = _logits().numpy()
    assert np.array_equal(osm.sampling_probabilities(x, 1.0, 1, 1.0),
                          osm.sampling_probabilities(x, 0.0, 0, 1.0))
    g = osm.sampling_probabilities(x, 0.0, 0, 1.0)
    assert np.array_equal(g.argmax(1), x.argmax(1)) and np.all(g.sum(1) == 1.0)


def test_oracle_truncation_keeps_relative_odds():
    x = _logits().numpy()
    full = osm.sampling_probabilities(x, 1.0, 0, 1.0)
    cut = osm.sampling_probabilities(x, 1.0, 4, 1.0)
    ratio = (cut[cut > 0] / full[cut > 0]).reshape(4, 4)
    assert np.allclose(ratio, ratio[:, :1])


# ------------------------------------------------------ library vs oracle


@pytest.mark.parametrize("params", [
    SamplingParams(), SamplingParams(temperature=0.0), SamplingParams(temperature=0.25),
    SamplingParams(temperature=2.0), SamplingParams(top_k=3), SamplingParams(top_k=VOCAB * 10),
    SamplingParams(top_p=0.5), SamplingParams(top_p=1e-6), SamplingParams(temperature=0.8, top_k=8, top_p=0.9),
], ids=str)
def test_probabilities_match_the_oracle(params):
    x = _logits(6, seed=3)
    got = sampling_probabilities(x, params)
    assert got.dtype == torch.float32
    assert np.allclose(got.numpy(), _oracle(x, params), rtol=0, atol=2e-6)
    assert torch.allclose(got.sum(1), torch.ones(6), atol=1e-5)


def test_each_row_takes_its_own_parameters():
    x = _logits(4, seed=5)
    rows = [SamplingParams(temperature=0.0), SamplingParams(), SamplingParams(top_k=2),
            SamplingParams(top_p=0.5)]
    got = sampling_probabilities(x, rows)
    for r, params in enumerate(rows):
        assert np.allclose(got[r:r + 1].numpy(), _oracle(x[r:r + 1], params), atol=2e-6)


def test_validation_and_shapes():
    for kwargs, match in (({"temperature": -0.1}, "temperature"), ({"top_k": -1}, "top_k"),
                          ({"top_p": 0.0}, "top_p"), ({"top_p": 1.5}, "top_p")):
        with pytest.raises(ValueError, match=match):
            SamplingParams(**kwargs)
    with pytest.raises(ValueError, match="expected B x V"):
        sampling_probabilities(torch.randn(VOCAB), SamplingParams())
    with pytest.raises(ValueError, match="for a batch of 4"):
        sampling_probabilities(_logits(), [SamplingParams()] * 3)
    tokens = sample(_logits(), SamplingParams())
    assert tokens.shape == (4,) and tokens.dtype == torch.int64


def test_draws_are_reproducible_and_stay_in_the_kept_set():
    x = _logits(8, seed=9)
    params = SamplingParams(top_k=3, top_p=0.9)
    kept = sampling_probabilities(x, params) > 0
    seen = set()
    for seed in range(30):
        a = sample(x, params, generator=torch.Generator().manual_seed(seed))
        b = sample(x, params, generator=torch.Generator().manual_seed(seed))
        assert torch.equal(a, b)
        assert kept[torch.arange(8), a].all()
        seen.add(tuple(a.tolist()))
    assert len(seen) > 1
    greedy = sample(x, [SamplingParams(temperature=0.0), SamplingParams(temperature=2.0)] * 4,
                    generator=torch.Generator().manual_seed(1))
    assert torch.equal(greedy[0::2], x[0::2].argmax(1))


def test_bf16_logits_give_fp32_probabilities():
    x = _logits(2).to(torch.bfloat16)
    got = sampling_probabilities(x, SamplingParams(top_k=4))
    assert got.dtype == torch.float32 and torch.allclose(got.sum(1), torch.ones(2), atol=1e-6)
    assert np.allclose(got.numpy(), _oracle(x, SamplingParams(top_k=4)), atol=2e-6)
