"""The paged engine on the CPU (PyTorch path) against the dense float64 recompute.

The reference's engine tests (tests/test_engine.py:56-350) in this form: chunked and
unchunked prefill, many sequences sharing iterations, preemption under a pool too small
for everyone, an impossible pool, and no block leaks afterwards.
"""

from __future__ import annotations

import pytest
import torch

from engine_helpers import assert_tokens_match, make_engine, prompts, tiny_config
from mini_vllm.block import OutOfBlocks
from mini_vllm.model import random_weights
from mini_vllm.serve import SchedulerConfig
from oracle.qwen3_dense import generate_greedy

MAX_TOKENS = 8


@pytest.fixture(scope="module")
def model():
    config = tiny_config()
    return config, random_weights(config, seed=3)


@pytest.fixture(scope="module")
def reference(model):
    config, weights = model
    ps = prompts(6, 3, 40, config.vocab_size, seed=1)
    return ps, [generate_greedy(config, weights, p, MAX_TOKENS) for p in ps]


@pytest.mark.parametrize("sched", [
    SchedulerConfig(),                                                 # everything in one pass
    SchedulerConfig(max_batched_tokens=16, chunk_size=8),             # chunked, piggybacked
    SchedulerConfig(max_batched_tokens=64, enable_chunked_prefill=False),
    SchedulerConfig(max_sequences=2, max_batched_tokens=24, chunk_size=5),
], ids=["one-pass", "chunked", "unchunked", "two-at-a-time"])
def test_engine_matches_dense_recompute(model, reference, sched):
    config, weights = model
    ps, want = reference
    engine = make_engine(config, weights, sched=sched)
    got = engine.generate(ps, MAX_TOKENS)
    for i, (g, (tok, logits)) in enumerate(zip(got, want)):
        assert_tokens_match(g, tok, logits, tie_tol=1e-4, msg=f"prompt {i}")
    engine.model.manager.check_no_leaks()
    assert engine.model.manager.num_free_blocks == engine.model.manager.num_blocks


def test_preemption_under_a_small_pool_still_matches(model, reference):
    config, weights = model
    ps, want = reference
    engine = make_engine(config, weights, num_blocks=6, block_size=8,
                         sched=SchedulerConfig(max_batched_tokens=32, chunk_size=16))
    got = engine.generate(ps, MAX_TOKENS)
    assert engine.stats.preemptions > 0, "the pool was meant to force preemption"
    for i, (g, (tok, logits)) in enumerate(zip(got, want)):
        assert_tokens_match(g, tok, logits, tie_tol=1e-4, msg=f"prompt {i}")
    engine.model.manager.check_no_leaks()


def test_a_pool_that_cannot_hold_one_sequence_raises(model):
    config, weights = model
    engine = make_engine(config, weights, num_blocks=2, block_size=4)
    with pytest.raises(OutOfBlocks):
        engine.generate([list(range(40))], 4)


def test_stats_count_what_ran(model):
    config, weights = model
    engine = make_engine(config, weights, sched=SchedulerConfig(max_batched_tokens=16, chunk_size=8))
    ps = prompts(3, 5, 20, config.vocab_size, seed=4)
    engine.generate(ps, 5)
    s = engine.stats
    assert s.generated_tokens == 15
    assert s.prefill_tokens == sum(len(p) for p in ps)
    assert s.decode_tokens == 3 * 4
    assert s.decode_only_tokens <= s.decode_tokens


def test_logits_rows_are_each_sequences_last_position(model):
    """One row per sequence, at its own last computed position (test_engine.py:154-179)."""
    config, weights = model
    engine = make_engine(config, weights)
    ps = prompts(3, 4, 12, config.vocab_size, seed=7)
    seqs = [engine.add_request(p, 1) for p in ps]
    engine.step()
    for seq, p in zip(seqs, ps):
        tok, _ = generate_greedy(config, weights, p, 1)
        assert seq.output == tok


def test_use_cuda_model_on_cpu_tensors_equals_the_pytorch_path(model):
    """Port of the reference's tests/test_qwen3_cached.py:335-350 to the paged model:
    a model built with ``use_cuda=True`` on CPU tensors falls back op by op and gives
    exactly the ``use_cuda=False`` model's logits and tokens (the same model object
    serves CPU tests and GPU serving)."""
    from mini_vllm.kernels import ops
    from mini_vllm.serve.batch import ForwardBatch

    config, weights = model
    ps = prompts(3, 4, 20, config.vocab_size, seed=11)
    logits = {}
    for use_cuda in (False, True):
        engine = make_engine(config, weights, use_cuda=use_cuda)
        seqs = [engine.add_request(p, 4) for p in ps]
        out = engine.scheduler.schedule()
        batch = ForwardBatch.from_scheduled(out.scheduled, engine.model.manager)
        logits[use_cuda] = engine.model(batch)
        engine.scheduler.commit(out, ops.argmax(logits[use_cuda]).tolist())
        while engine.scheduler.has_work:
            engine.step()
        logits[use_cuda, "tokens"] = [s.output for s in seqs]
    assert torch.equal(logits[True], logits[False])
    assert logits[True, "tokens"] == logits[False, "tokens"]
    assert "declined calls" in ops.dispatch_report(True)


def test_cached_dense_recompute_equals_the_full_recompute(model):
    """The oracle's KV-cached greedy loop (used at the 0.6B shape, where recomputing
    every step is too slow) against its full recompute: same tokens, logits to 1e-12."""
    from oracle.qwen3_dense import generate_greedy_cached

    config, weights = model
    for p in prompts(3, 1, 30, config.vocab_size, seed=12):
        tok, logits = generate_greedy(config, weights, p, 6)
        tok_c, logits_c = generate_greedy_cached(config, weights, p, 6)
        assert tok == tok_c
        for a, b in zip(logits, logits_c):
            assert (a - b).abs().max() < 1e-12


@pytest.mark.parametrize("num_blocks", [7, 8])
def test_two_long_prompts_do_not_evict_each_other_forever(num_blocks):
    """Regression: with a victim readmitted in the iteration that evicted it, two long
    prompts in a 7- or 8-page pool kept evicting each other, each restarting from token
    zero, and the engine never finished. A victim now waits one iteration."""
    from mini_vllm.block import BlockManager
    from mini_vllm.serve import Scheduler
    from mini_vllm.serve.sequence import Sequence

    manager = BlockManager(num_blocks, 8, 1, 1, 8, torch.float32)
    sched = Scheduler(SchedulerConfig(max_batched_tokens=32, chunk_size=16), manager)
    lens = [36, 21, 29, 35, 12, 10]
    seqs = [Sequence(i, list(range(n)), 8) for i, n in enumerate(lens)]
    for s in seqs:
        sched.add(s)
    preempted = 0
    for _ in range(500):
        if not sched.has_work:
            break
        out = sched.schedule()
        preempted += len(out.preempted)
        sched.commit(out, [0] * len(out.scheduled))
    assert not sched.has_work, "the scheduler did not finish"
    assert preempted > 0 and all(len(s.output) == 8 for s in seqs)
    manager.check_no_leaks()


def test_sampled_requests_are_reproducible_and_greedy_ones_unchanged(model):
    """Requests with their own sampling parameters beside greedy ones (reference
    serve/engine.py:252-330): the greedy requests still equal the dense recompute,
    the sampled ones repeat exactly under the same generator seed and differ under
    another, and every token is in the vocabulary."""
    from mini_vllm.sampler import SamplingParams

    config, weights = model
    ps = prompts(6, 3, 30, config.vocab_size, seed=1)
    hot = SamplingParams(temperature=1.5, top_k=50, top_p=0.95)
    params = [None, hot, None, hot, SamplingParams(temperature=0.0), hot]

    def run(seed):
        engine = make_engine(config, weights)
        engine.generator = torch.Generator().manual_seed(seed)
        return engine.generate(ps, MAX_TOKENS, params)

    first, again, other = run(5), run(5), run(6)
    assert first == again and first != other
    for i in (0, 2, 4):
        tok, logits = generate_greedy(config, weights, ps[i], MAX_TOKENS)
        assert_tokens_match(first[i], tok, logits, tie_tol=1e-4, msg=f"greedy request {i}")
    assert all(0 <= t < config.vocab_size for g in first for t in g)
    with pytest.raises(ValueError, match="sampling params"):
        make_engine(config, weights).generate(ps, 2, [hot])


class _EagerGraphs:
    """Stands in for DecodeGraphs.run on the CPU: the same input rule (a sequence in
    ``prev_rows`` takes ``prev_tokens[row]`` as its input token, every other row the
    host's token) and the same output (the logits, their argmax written to the head of
    ``prev_tokens`` as a replay's last launch does) without capturing a graph, so the
    engine's bookkeeping of which sampled tokens the next iteration may gather is
    checked here. Records every (sequence, position, token fed)."""

    def __init__(self, graphs):
        self.graphs = graphs
        self.fed = []

    def __call__(self, scheduled):
        from dataclasses import replace

        from mini_vllm.serve.batch import ForwardBatch

        g = self.graphs
        batch = ForwardBatch.from_scheduled(scheduled, g.model.manager, "cpu")
        ids = batch.input_ids.clone()
        for i, (seq, _) in enumerate(scheduled):
            row = g.prev_rows.get(seq.seq_id, -1)
            if row >= 0:
                ids[i] = g.prev_tokens[row]
            self.fed.append((seq, seq.num_computed_tokens, int(ids[i])))
        g.replays += 1
        logits = g.model(replace(batch, input_ids=ids))
        g.prev_tokens[:len(scheduled)].copy_(logits.argmax(dim=-1))
        return logits


@pytest.mark.parametrize("lengths,sched", [
    ((9, 17), SchedulerConfig(max_batched_tokens=24, chunk_size=8)),   # last chunk 1 token
    # two rows decode, so a 3-token budget leaves the third prompt 1-token chunks
    ((2, 2, 12), SchedulerConfig(max_batched_tokens=3, chunk_size=8)),
], ids=["chunk-plus-one", "one-token-chunks"])
def test_decode_rows_gather_only_committed_tokens(model, lengths, sched):
    """Iterations whose rows are all one token go to the decode graphs even when a row
    is a prompt chunk that does not finish its prompt; that row's sampled token is
    discarded, so the next iteration must not feed it back as the sequence's input.
    Every token fed to a replay is the sequence's token at that position, and the
    tokens match the float64 recompute (the graph replay is emulated eagerly)."""
    config, weights = model
    g = torch.Generator().manual_seed(21)
    ps = [torch.randint(0, config.vocab_size, (n,), generator=g).tolist() for n in lengths]
    engine = make_engine(config, weights, sched=sched, use_graphs=True)
    replay = engine.graphs.run = _EagerGraphs(engine.graphs)
    got = engine.generate(ps, MAX_TOKENS)
    assert engine.graphs.replays > 0
    for seq, pos, token in replay.fed:
        assert seq.tokens(pos, 1)[0] == token, (seq.seq_id, pos)
    for i, (p, g) in enumerate(zip(ps, got)):
        tok, logits = generate_greedy(config, weights, p, MAX_TOKENS)
        assert_tokens_match(g, tok, logits, tie_tol=1e-4, msg=f"prompt {i}")


@pytest.mark.parametrize("sched", [SchedulerConfig(), SchedulerConfig(max_batched_tokens=24, chunk_size=8)],
                         ids=["one-pass", "chunked"])
def test_fp8_kv_engine_matches_the_fp8_dense_recompute(sched):
    """An fp8-e4m3 KV pool on the PyTorch path against the float64 dense recompute whose
    K/V go through oracle/kv_write.py's quantising write (oracle/qwen3_dense.py with
    kv_fp8): the same greedy tokens up to genuine near-ties. Weights of std 0.3 make
    the tokens depend on the quantisation: the recompute without it diverges on some
    prompts, so agreeing with the fp8 one is a real check. The engine's chunks of 8
    leave pages half written between chunks (their scale grows on the next write), the
    recompute writes each prompt whole: the same values except where a grown scale
    re-rounds, which the tie tolerance covers."""
    from oracle.qwen3_dense import DenseQwen3

    config = tiny_config()
    weights = random_weights(config, seed=3, std=0.3)
    ps = prompts(6, 3, 40, config.vocab_size, seed=4)
    engine = make_engine(config, weights, sched=sched, kv_dtype=torch.float8_e4m3fn)
    got = engine.generate(ps, MAX_TOKENS)
    fp8 = [DenseQwen3(config, weights, kv_fp8=True).generate(p, MAX_TOKENS) for p in ps]
    for i, (g, (tok, logits)) in enumerate(zip(got, fp8)):
        assert_tokens_match(g, tok, logits, tie_tol=1e-3, msg=f"prompt {i}")
    plain = DenseQwen3(config, weights)
    assert any(plain.generate(p, MAX_TOKENS)[0] != t for p, (t, _) in zip(ps, fp8))
    engine.model.manager.check_no_leaks()
