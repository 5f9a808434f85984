"""The read-only HBM probe behind bench.py's bandwidth ceiling (``mvllm_read_probe``)
on the MI355X: it must read every page it is given exactly once, whichever order, or
the ceiling it reports is not a read of those bytes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("page_bytes", [4096, 32768, 65536])
@pytest.mark.parametrize("order", ["address", "shuffled"])
def test_every_word_is_read_once(extension, device, page_bytes, order):
    """The XOR of every lane's folded word equals the XOR of the whole buffer: each
    word reached exactly one lane once (a page read twice cancels itself out, a page
    skipped leaves its words out)."""
    pages = 96
    base = torch.randint(-2**31, 2**31 - 1, (pages * page_bytes // 4,), dtype=torch.int32,
                         device=device)
    ids = None
    if order == "shuffled":
        ids = torch.randperm(pages, generator=torch.Generator().manual_seed(1)).to(torch.int32).to(device)
    for wgs in (1, 7, 256):
        sink = torch.zeros(wgs * 256, dtype=torch.int32, device=device)
        extension.read_probe(base, page_bytes, ids, wgs, sink)
        torch.cuda.synchronize()
        want = np.bitwise_xor.reduce(base.cpu().numpy().view(np.uint32))
        got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
        assert got == want, (order, wgs)
