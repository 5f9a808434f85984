"""Pure-decode iterations replayed from captured HIP graphs.

A decode iteration of the paged model is ~15 ops per layer; dispatched one by one from
Python it costs several milliseconds of host time for about one millisecond of GPU work
(the reference lists this as the engine's next bottleneck, serve/batch.py:286-347,
runner.py:65-66). Every op of a decode step reads its per-iteration inputs from device
tensors -- token ids, positions, slots, context lengths, block tables -- and the host
integers the launches depend on (batch size, an upper bound on the context) can be held
fixed, so one captured graph serves every decode step of a given shape:

* graphs are keyed by (batch bucket, table width): the batch is padded up to a bucket
  with dummy sequences (one token of context in a reserved page, rows discarded), and
  the block-table width is rounded up to a multiple of 64 pages;
* before a replay, the iteration's metadata is packed into one pinned host buffer and
  copied into the graph's static input tensors with one host-to-device copy;
* greedy sampling (argmax) is the graph's last launch and writes the sampled tokens
  straight into a device buffer every graph reads (:attr:`DecodeGraphs.prev_tokens`;
  other sampling runs after the replay on its logits and :meth:`DecodeGraphs.keep`
  copies its tokens there; keep records which rows were committed); a sequence whose token
  from the previous iteration was committed takes its next input token from there, so
  the host need not have read that token yet: the engine schedules and packs the next
  decode step while the GPU runs this one. The model's first launch (the embedding
  lookup with the first block's input norm) picks each row's token: row i takes
  ``prev_tokens[gather[i]]``, its row of the previous replay, or with ``gather[i] = -1``
  its host id (the batch's ``input_source``: host ids, gather, prev_tokens).

The paged-attention plan in stream mode depends only on the batch size and the bound on
max_context_len, so the kernels launched inside a graph stay valid for every replay;
they read the real context lengths from the static buffers.
"""

from __future__ import annotations

import torch

from mini_vllm.kernels import ops

from mini_vllm.serve.batch import PADDING_BLOCK, ForwardBatch

__all__ = ["DecodeGraphs"]

BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256)
TABLE_QUANTUM = 64  # pages


class _Captured:
    def __init__(self, model, batch_size: int, width: int, dummy_block: int, device,
                 prev: torch.Tensor) -> None:
        p = model.manager.block_size
        self.batch_size, self.width = batch_size, width
        b = batch_size
        i32 = dict(dtype=torch.int32, device=device)
        i64 = dict(dtype=torch.int64, device=device)
        # Dynamic inputs, one device buffer written by one copy from one pinned host
        # buffer: int64 [ids | gather | positions], then int32 [context | slots | tables].
        # Row i's input token is prev[gather[i]], the token sampled for it by the previous
        # replay (still on the device), or with gather[i] = -1 its id from the host.
        n64, n32 = 3 * b, 2 * b + b * width
        self.dyn = torch.zeros(8 * n64 + 4 * n32, dtype=torch.uint8, device=device)
        self.host = torch.zeros(8 * n64 + 4 * n32, dtype=torch.uint8, pin_memory=True)
        dyn64 = self.dyn[:8 * n64].view(torch.int64)
        dyn32 = self.dyn[8 * n64:].view(torch.int32)
        self.prev = prev
        self.batch = ForwardBatch(
            input_ids=dyn64[:b],  # the host's ids (0 in gathered rows): see input_source
            positions=dyn64[2 * b:3 * b],
            cu_seqlens_q=torch.arange(b + 1, **i32),
            seq_lens=torch.ones(b, **i32),
            context_lens=dyn32[:b],
            slot_mapping=dyn32[b:2 * b],
            block_tables=dyn32[2 * b:].view(b, width),
            last_row_indices=torch.arange(b, **i64),
            max_query_len=1,
            max_context_len=width * p,
            seq_ids=tuple(range(b)),
            input_source=(dyn64[:b], dyn64[b:2 * b], prev),
        )
        self.dummy_block = dummy_block
        self.model = model
        self.graph = None
        self.logits = None
        self.workspaces: list[torch.Tensor] = []  # kernel workspaces the graph names
        # numpy views of the pinned buffer, written in place; each table row is
        # rewritten only when the block manager reports a change of that sequence's
        # table (row_keys: (seq_id, version), or None for a dummy row).
        self.np64 = self.host[:8 * n64].view(torch.int64).numpy()
        self.np32 = self.host[8 * n64:].view(torch.int32).numpy()
        self.row_keys: list = [()] * b
        self._copied = None  # event after the last copy out of the pinned buffer

    def fill(self, scheduled, gather: list[int] | None = None) -> None:
        b, w, p = self.batch_size, self.width, self.model.manager.block_size
        manager = self.model.manager
        if self._copied is not None:
            # the previous replay's copy must have read the pinned buffer before it is
            # rewritten (it normally has: it runs as that replay starts)
            self._copied.synchronize()
        ids, rows, pos = self.np64[:b], self.np64[b:2 * b], self.np64[2 * b:]
        ctx, slots = self.np32[:b], self.np32[b:2 * b]
        tables = self.np32[2 * b:].reshape(b, w)
        for i, (seq, _) in enumerate(scheduled):
            start = seq.num_computed_tokens
            g = gather[i] if gather is not None else -1
            # a gathered row's token may not have reached the host yet
            rows[i] = g if g >= 0 else -1
            ids[i] = seq.tokens(start, 1)[0] if g < 0 else 0
            pos[i] = start
            ctx[i] = start + 1
            table = manager.table(seq.seq_id)
            slots[i] = table[start // p] * p + start % p
            key = (seq.seq_id, manager.version(seq.seq_id))
            if self.row_keys[i] != key:
                tables[i, :len(table)] = table
                tables[i, len(table):] = PADDING_BLOCK
                self.row_keys[i] = key
        for i in range(len(scheduled), b):
            rows[i] = -1
            if self.row_keys[i] is not None:
                ids[i], pos[i], ctx[i], slots[i] = 0, 0, 1, self.dummy_block * p
                tables[i, 0] = self.dummy_block
                tables[i, 1:] = PADDING_BLOCK
                self.row_keys[i] = None
        self.dyn.copy_(self.host, non_blocking=True)
        if self.dyn.is_cuda:
            self._copied = torch.cuda.Event()
            self._copied.record()

    def _forward(self, sampled: torch.Tensor) -> torch.Tensor:
        logits = self.model(self.batch)
        ops.argmax(logits, use_cuda=self.model.use_cuda, out=sampled)
        return logits

    def capture(self) -> None:
        # Warm up on a side stream (allocator pools, BLAS handles, the kernels' per-stream
        # workspaces), then capture on that same stream.
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # (the warm-up's tokens go to a scratch buffer: the shared one still holds
            # the previous replay's, which this iteration's replay gathers)
            scratch = torch.empty(self.batch_size, dtype=torch.int64, device=self.prev.device)
            for _ in range(2):
                self._forward(scratch)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        recorder = _workspace_recorder(self.model)
        with recorder as workspaces, torch.cuda.graph(self.graph, stream=side):
            # The greedy tokens, into the head of the shared token buffer the next
            # replay gathers from (dummy rows' too, beyond the real ones: never gathered).
            self.logits = self._forward(self.prev[:self.batch_size])
        self.workspaces = list(workspaces)


class _NoRecorder:
    def __enter__(self):
        return []

    def __exit__(self, *exc):
        return False


def _workspace_recorder(model):
    """Records the kernel library's workspaces a capture names (nothing to record on
    the PyTorch path), so the graph keeps them alive."""
    if not model.use_cuda:
        return _NoRecorder()
    from mini_vllm.kernels.extension import load_extension

    return load_extension().recording_workspaces()


class DecodeGraphs:
    """Replays pure-decode iterations of ``model`` from captured graphs."""

    def __init__(self, model, max_batch: int = 32) -> None:
        self.model = model
        self.max_batch = max_batch
        self.device = model.weights["embedding"].device
        manager = model.manager
        # A page no sequence ever owns: the dummy rows of a padded batch write there.
        self._dummy_id = -1
        manager.allocate(self._dummy_id, 1)
        self.dummy_block = manager.table(self._dummy_id)[0]
        self.graphs: dict[tuple[int, int], _Captured] = {}
        self.replays = 0
        # The tokens sampled by the last replay: row i is the token of the sequence
        # prev_rows maps to i, read by the next replay's gather.
        self.prev_tokens = torch.zeros(max(BUCKETS), dtype=torch.int64, device=self.device)
        self.prev_rows: dict[int, int] = {}

    def supports(self, scheduled) -> bool:
        return 0 < len(scheduled) <= self.max_batch and all(n == 1 for _, n in scheduled)

    def run(self, scheduled) -> torch.Tensor:
        """Logits ``len(scheduled) x V`` for a pure-decode iteration; their argmax is in
        ``prev_tokens[:len(scheduled)]`` when the replay ends. A sequence that was in the
        previous replay, and whose token from it was handed to :meth:`keep`, reads that
        token on the device."""
        n = len(scheduled)
        bucket = next(b for b in BUCKETS if b >= n)
        widest = max(len(self.model.manager.table(s.seq_id)) for s, _ in scheduled)
        width = -(-widest // TABLE_QUANTUM) * TABLE_QUANTUM
        key = (bucket, width)
        gather = [self.prev_rows.get(s.seq_id, -1) for s, _ in scheduled]
        entry = self.graphs.get(key)
        if entry is None:
            entry = _Captured(self.model, bucket, width, self.dummy_block, self.device,
                              self.prev_tokens)
            entry.fill(scheduled, gather)
            entry.capture()
            self.graphs[key] = entry
        entry.fill(scheduled, gather)
        entry.graph.replay()
        self.replays += 1
        return entry.logits[:n]

    def keep(self, scheduled, tokens: torch.Tensor, committed) -> None:
        """The tokens just sampled for ``scheduled`` (device, one per row) and the rows
        ``committed`` whose token became its sequence's new last token: the next replay
        gathers its inputs from those rows only. A row whose token was discarded (a
        prompt chunk that did not reach the prompt's end, or a recompute chunk short of
        the sequence's end) is not kept: that sequence's next input is a token the host
        already has. ``tokens`` may already be the head of :attr:`prev_tokens` (the
        argmax wrote there): then nothing is copied."""
        n = len(scheduled)
        if tokens.data_ptr() != self.prev_tokens.data_ptr() or tokens.numel() != n:
            self.prev_tokens[:n].copy_(tokens)
        self.prev_rows = {scheduled[i][0].seq_id: i for i in committed}

    def invalidate(self) -> None:
        """An iteration ran outside the graphs: no device-held token is current."""
        self.prev_rows = {}
