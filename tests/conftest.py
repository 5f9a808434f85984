"""Shared fixtures and comparison helpers.

Markers: ``gpu`` (needs an MI355X; everything else runs on the CPU). The package lives
in ``mini-vllm_amd/`` (a directory name that is not an import name), so it is put on
``sys.path`` here, as a user of the library would.
"""

from __future__ import annotations

import random
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
for path in (REPO / "mini-vllm_amd", REPO):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

SEED = 1234

# Tolerances. Paged attention is compared with the fp32 oracle (oracle/) by max-abs
# error, at the bounds the hot path is specified to: 2e-2 for bf16, 6e-2 for an fp8
# KV cache; fp32 and fp16 get their own (fp32: accumulation-order noise only).
ATTN_ATOL = {
    torch.float32: 2e-5,
    torch.float16: 1e-2,
    torch.bfloat16: 2e-2,
    torch.float8_e4m3fn: 6e-2,
}


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (run with -m gpu)")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(autouse=True)
def seeded():
    torch.manual_seed(SEED)
    random.seed(SEED)


@pytest.fixture(autouse=True)
def strict_kernels_on_gpu(request):
    """GPU tests run the seam in strict mode: a ``use_cuda=True`` call the kernels
    decline raises instead of passing on the PyTorch path, so no GPU test can pass on
    a fallback. Tests of the fallback itself switch it off for their block."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    from mini_vllm.kernels import ops

    previous = ops.set_strict(True)
    try:
        yield
    finally:
        ops.set_strict(previous)


@pytest.fixture(scope="session")
def device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda")


@pytest.fixture(scope="session")
def extension(device):
    from mini_vllm.kernels.extension import load_extension

    return load_extension()


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def assert_max_abs(actual: torch.Tensor, expected: torch.Tensor, atol: float, msg: str = "") -> None:
    assert actual.shape == expected.shape, f"{msg} shape {tuple(actual.shape)} != {tuple(expected.shape)}"
    a = actual.detach().double().cpu()
    assert torch.isfinite(a).all(), f"{msg} non-finite output"
    err = max_abs(actual, expected)
    assert err <= atol, f"{msg} max-abs error {err:.3e} > {atol:.1e}"
