"""The prefill projections through the library's hipBLASLt entry (``mvllm_blas_linear``,
``ops.linear`` / ``linear_split`` at prefill sizes) on the MI355X.

The product is hipBLASLt's (fp32 accumulation, one rounding to the output dtype): each
output must lie within one ulp of its float64 value plus the fp32 accumulation error
(bounded by K x 2^-23 x sum |x_i w_i| for any summation order), and agree with torch's
own product (the same library, possibly another algorithm) within two such bounds."""

from __future__ import annotations

import pytest
import torch

from mini_vllm.kernels import ops

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]  # Qwen3-0.6B's projections


def _eps(dtype) -> float:
    return 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11


def _bound(x, w, dtype):
    ref = x.double() @ w.double().T
    mag = x.double().abs() @ w.double().abs().T
    k = x.shape[1]
    return ref, _eps(dtype) * ref.abs() + k * 2.0**-23 * mag + 2.0**-60


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [65, 300, 1460, 2048])
def test_matches_float64_and_torch(extension, device, dtype, m):
    gen = torch.Generator().manual_seed(m)
    for n, k in SHAPES:
        x = torch.randn(m, k, generator=gen).to(dtype).to(device)
        w = (torch.randn(n, k, generator=gen) * 0.02).to(dtype).to(device)
        y = extension.blas_linear(x, w)
        assert y is not None and y.shape == (m, n) and y.dtype == dtype
        theirs = x @ w.t()
        torch.cuda.synchronize()
        ref, bound = _bound(x, w, dtype)
        err = (y.double() - ref).abs()
        assert (err <= bound).all(), f"{(m, n, k)}: off by {(err / bound).max().item():.2f} bounds"
        assert ((y.double() - theirs.double()).abs() <= 2 * bound).all(), (m, n, k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,k", SHAPES)
def test_every_row_count_of_the_buckets(extension, device, n, k, dtype):
    """m values share one algorithm per 128-row bucket (chosen at the bucket's largest,
    odd, m, timed at the bucket's first call): every m - bucket edges, odd and even,
    from 65 to 2048 - stays within the bound, the algorithm not assuming anything of m;
    for every shape of the model and both 16-bit dtypes."""
    gen = torch.Generator().manual_seed(n + k)
    x = torch.randn(2048, k, generator=gen).to(dtype).to(device)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dtype).to(device)
    ms = sorted(set(list(range(65, 2049, 61)) + [127, 128, 129, 255, 256, 257, 1023, 1024,
                                                 1025, 1535, 1536, 2047, 2048]))
    for m in ms:
        y = extension.blas_linear(x[:m], w)
        ref, bound = _bound(x[:m], w, dtype)
        err = (y.double() - ref).abs()
        assert (err <= bound).all(), f"m={m}: off by {(err / bound).max().item():.2f} bounds"


def test_the_kept_algorithm_is_the_fastest_candidate(extension, device):
    """A bucket's first call times the heuristic's candidates and keeps the fastest
    (never slower than the heuristic's first, which is one of them); every m of the
    bucket then reuses it, and its products stay within the bound."""
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(1500, 1024, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(6144, 1024, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    extension.blas_linear(x[:1407], w)  # bucket 10 (m 1280-1407)
    first = extension.blas_choice(1407, 6144, 1024, torch.bfloat16)
    assert first["candidates"] >= 1 and first["timed"] >= 1
    assert 0 <= first["chosen"] < first["candidates"]
    assert first["chosen_us"] <= first["first_us"]
    for m in (1281, 1300, 1406):
        y = extension.blas_linear(x[:m], w)
        assert extension.blas_choice(m, 6144, 1024, torch.bfloat16) == first
        ref, bound = _bound(x[:m], w, torch.bfloat16)
        assert ((y.double() - ref).abs() <= bound).all(), m


def test_a_first_call_under_graph_capture(extension, device):
    """A shape first called while its stream is being captured cannot be timed (no host
    wait inside a capture): it keeps the heuristic's first, untimed, and the replayed
    graph gives the eager product's bits, replay after replay."""
    gen = torch.Generator().manual_seed(12)
    m, n, k = 1024 + 77, 768, 1536  # an (n, k) no other test calls: its bucket is new
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        y = extension.blas_linear(x, w)
    choice = extension.blas_choice(m, n, k, torch.bfloat16)
    assert choice["timed"] == 0 and choice["chosen"] == 0 and choice["first_us"] == -1
    eager = extension.blas_linear(x, w)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


def test_kept_shapes_and_a_second_stream(extension, device):
    """A repeated shape reuses its kept set-up (no new entry); a new one adds one; a call
    on another stream (its own workspace) gives the same bits as on the default stream."""
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(777, 1024, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(4096, 1024, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    first = extension.blas_linear(x, w)
    kept = extension.blas_plans_cached()
    for _ in range(3):
        assert torch.equal(extension.blas_linear(x, w), first)
    assert extension.blas_plans_cached() == kept
    extension.blas_linear(x[:500], w)
    assert extension.blas_plans_cached() == kept + 1
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        other = extension.blas_linear(x, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(other, first)


def test_ops_route_prefill_products_through_it(extension, device):
    """ops.linear and ops.linear_split at prefill sizes run the library's entry (a new
    shape adds a kept entry) and give its bits; fp32 and host tensors take torch's
    product."""
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(999, 1024, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(4096, 1024, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    pw = ops.pack_weight(w, use_cuda=True)
    before = extension.blas_plans_cached()
    y = ops.linear(x, pw, use_cuda=True)
    assert extension.blas_plans_cached() == before + 1
    assert torch.equal(y, extension.blas_linear(x, w))
    q, k, v = ops.linear_split(x, pw, (2048, 1024, 1024), use_cuda=True, views=True)
    assert torch.equal(torch.cat([q, k, v], dim=-1), y)
    xf, wf = x.float(), w.float()
    assert torch.equal(ops.linear(xf, wf, use_cuda=True), xf @ wf.t())
    assert not extension.blas_linear_supported(xf, wf)
    with pytest.raises(RuntimeError, match="not served"):
        extension.blas_linear(xf, wf)
    with pytest.raises(RuntimeError, match="not served"):
        extension.blas_linear(x[:, :512], w[:, :512])  # strided, not contiguous


def test_a_sweep_adds_faster_candidates(extension, device):
    """``blas_tune`` times every algorithm at one row count and leaves y = x w^T; the
    choices made after it include its fastest (a kept index past the heuristic's 16 is
    one of them) and are never slower than the heuristic's first; products stay within
    the bound at the swept m and at other buckets (whose m the kept algorithms are
    checked against before they are timed)."""
    gen = torch.Generator().manual_seed(13)
    n, k = 1536, 512  # a shape no other test calls
    x = torch.randn(1024, k, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    before = extension.blas_linear(x[:700], w)
    timed = extension.blas_tune(x, w)
    assert timed > 16
    for m in (700, 1024, 333):
        y = extension.blas_linear(x[:m], w)
        ref, bound = _bound(x[:m], w, torch.bfloat16)
        assert ((y.double() - ref).abs() <= bound).all(), m
        choice = extension.blas_choice(m, n, k, torch.bfloat16)
        assert choice["timed"] >= 1 and choice["chosen_us"] <= choice["first_us"]
        if m == 1024:  # the swept shape itself: all 12 kept algorithms serve it
            assert choice["candidates"] >= 13, choice
    assert ((extension.blas_linear(x[:700], w).double() - before.double()).abs()
            <= 2 * _bound(x[:700], w, torch.bfloat16)[1]).all()


def test_a_sweep_is_refused_under_capture(extension, device):
    x = torch.randn(256, 512, device=device).to(torch.bfloat16)
    w = torch.randn(512, 512, device=device).to(torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capturing"):
        with torch.cuda.graph(graph, stream=side):
            extension.blas_tune(x, w)
