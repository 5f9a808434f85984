"""Greedy sampling kernel (``ops.argmax`` / ``mvllm_argmax``) on the MI355X (``-m gpu``).

The reference's greedy rows take ``logits.argmax(dim=-1)`` (mini_vllm/sampler.py:
135-141). Index work is bit-exact: the kernel must return torch's indices, including
its order on ties (first index), signed zeros (equal) and NaN (above every number).
"""

from __future__ import annotations

import pytest
import torch

from mini_vllm.kernels import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,vocab", [(1, 1), (3, 7), (4, 8), (32, 151936), (65, 1000),
                                        (5, 16385), (2, 300001), (1, 1048576)])
def test_matches_torch_argmax(extension, device, rows, vocab, dtype):
    gen = torch.Generator().manual_seed(rows * 31 + vocab)
    logits = torch.randn(rows, vocab, generator=gen).to(dtype).cuda()
    assert torch.equal(extension.argmax(logits), logits.argmax(dim=-1))


def test_ties_signed_zeros_and_nan(extension, device):
    """Equal maxima: the first index; -0 == +0 (the earlier zero wins); NaN beats every
    number and the first NaN wins; -inf rows and a row of one value."""
    x = torch.full((7, 50), -1.0)
    x[0, [5, 9, 40]] = 3.0                      # ties -> 5
    x[1, :] = -0.5
    x[1, 12], x[1, 30] = -0.0, 0.0              # -0 first, then +0: equal -> 12
    x[2, 30], x[2, 12] = -0.0, 0.0              # +0 first at 12 -> 12
    x[3, 44], x[3, 7], x[3, 8] = float("nan"), 1e30, float("nan")  # first NaN -> 8
    x[4, :] = float("-inf")                     # all -inf -> 0
    x[5, 49] = float("inf")                     # inf -> 49
    x[6, :] = 2.5                               # constant -> 0
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        logits = x.to(dtype).cuda()
        got = extension.argmax(logits)
        assert torch.equal(got, logits.argmax(dim=-1)), dtype
        assert got.tolist() == [5, 12, 12, 8, 0, 49, 0]


def test_strided_rows_and_ops_dispatch(extension, device):
    """Rows farther apart than their length (a narrowed logits buffer) and ``ops.argmax``
    routing: the kernel for 2-D f32/f16/bf16 rows, torch otherwise."""
    base = torch.randn(9, 1200, dtype=torch.bfloat16, device="cuda")
    view = base[:, 100:1100]
    assert not view.is_contiguous()
    assert torch.equal(extension.argmax(view), view.argmax(dim=-1))
    assert torch.equal(ops.argmax(view, use_cuda=True), view.argmax(dim=-1))
    x3 = torch.randn(2, 3, 40, device="cuda")
    assert torch.equal(ops.argmax(x3, use_cuda=True), x3.argmax(dim=-1))
    xd = torch.randn(4, 40, device="cuda", dtype=torch.float64)
    assert torch.equal(ops.argmax(xd, use_cuda=True), xd.argmax(dim=-1))
    with pytest.raises(RuntimeError, match="contiguous rows"):
        extension.argmax(base.t())


# ------------------------------------------------- temperature / top-k / top-p


def _oracle_probs(logits, params):
    from oracle import sampler as osm

    return torch.from_numpy(osm.sampling_probabilities(
        logits.float().cpu().numpy(), params.temperature, params.top_k, params.top_p)).float()


@pytest.mark.parametrize("params", [
    "greedy", "t1", "t0.7_k50", "t1.2_p0.9", "t0.8_k8_p0.9", "p1e-6"])
def test_device_sampling_probabilities_match_the_oracle(device, params):
    """At the Qwen3 vocabulary (151936) with bf16 logits, on the device, against the
    float64 oracle (ties, which bf16 logits make common, in vocabulary order on both
    sides)."""
    from mini_vllm.sampler import SamplingParams, sampling_probabilities

    sp = {"greedy": SamplingParams(temperature=0.0), "t1": SamplingParams(),
          "t0.7_k50": SamplingParams(temperature=0.7, top_k=50),
          "t1.2_p0.9": SamplingParams(temperature=1.2, top_p=0.9),
          "t0.8_k8_p0.9": SamplingParams(temperature=0.8, top_k=8, top_p=0.9),
          "p1e-6": SamplingParams(top_p=1e-6)}[params]
    gen = torch.Generator().manual_seed(17)
    logits = (torch.randn(8, 151936, generator=gen) * 3).to(torch.bfloat16).to(device)
    got = sampling_probabilities(logits, sp)
    assert got.is_cuda and got.dtype == torch.float32
    want = _oracle_probs(logits, sp)
    assert torch.equal(got.cpu() > 0, want > 0), "kept sets differ"
    assert torch.allclose(got.cpu(), want, rtol=1e-4, atol=1e-7)


def test_device_draws_are_reproducible_under_a_cuda_generator(device):
    from mini_vllm.sampler import SamplingParams, sample, sampling_probabilities

    logits = torch.randn(32, 151936, device=device, dtype=torch.bfloat16)
    rows = [SamplingParams(temperature=0.0), SamplingParams(temperature=1.0, top_k=40, top_p=0.9)] * 16
    kept = sampling_probabilities(logits, rows) > 0
    draws = []
    for seed in (3, 3, 4):
        g = torch.Generator(device=device).manual_seed(seed)
        draws.append(sample(logits, rows, generator=g))
    assert torch.equal(draws[0], draws[1]) and not torch.equal(draws[0], draws[2])
    for d in draws:
        assert d.is_cuda and bool(kept[torch.arange(32, device=device), d].all())
        assert torch.equal(d[0::2], logits[0::2].argmax(-1))


def test_device_draw_frequencies_follow_the_distribution(device):
    """20000 draws of one 8-token row at temperature 0.8 with top-k 6: every kept
    token's frequency within 4 standard errors of its probability, none outside."""
    import math

    from mini_vllm.sampler import SamplingParams, sample, sampling_probabilities

    draws = 20000
    row = torch.tensor([[2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -2.0]], device=device)
    sp = SamplingParams(temperature=0.8, top_k=6)
    p = sampling_probabilities(row, sp)[0].cpu()
    tokens = sample(row.expand(draws, -1).contiguous(), sp,
                    generator=torch.Generator(device=device).manual_seed(0))
    freq = torch.bincount(tokens.cpu(), minlength=8).double() / draws
    assert float(freq[6:].sum()) == 0.0
    for t in range(6):
        se = math.sqrt(float(p[t]) * (1 - float(p[t])) / draws)
        assert abs(float(freq[t]) - float(p[t])) < 4 * se, f"token {t}"


def test_writes_a_given_output(extension, device):
    """``out``: the indices land in the caller's int64 tensor (a view into a larger
    buffer, as the decode graphs pass), the rest of the buffer untouched; a wrong dtype
    or length is refused."""
    gen = torch.Generator().manual_seed(11)
    logits = torch.randn(5, 151936, generator=gen).to(torch.bfloat16).cuda()
    buf = torch.full((12,), -7, dtype=torch.int64, device="cuda")
    got = ops.argmax(logits, use_cuda=True, out=buf[:5])
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(buf[:5], logits.argmax(dim=-1)) and (buf[5:] == -7).all()
    with pytest.raises(RuntimeError, match="int64"):
        extension.argmax(logits, out=torch.empty(5, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="int64"):
        extension.argmax(logits, out=buf[:4])
