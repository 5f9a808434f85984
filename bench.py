"""Paged-attention hot-path benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extras] [--no-cpu]

A "step" is one ``ops.paged_attention(use_cuda=True)`` call over BASELINE config 2:
paged decode, bf16, batch 64, context lengths U[512, 4096] (seed 0), GQA 16q/8kv,
D=128, 16-token pages, shuffled block ids, pool = pages + 10%. Inputs are resident in
HBM before timing. Several copies of the pools are rotated so each step streams its
K/V from HBM rather than from the 256 MB Infinity Cache (config 2's K+V is ~0.6 GB).

``value`` is the algorithmic K+V bytes of one step (every visible key row read once,
the reference's definition, mini_vllm/bench.py:643) divided by the mean step time,
W warmup steps then K steps between two synchronizations, timed with HIP events on
the stream the kernels run on. Extras (configs 3 and 4, a device copy ceiling) are
reported in the same JSON line. ``cpu_baseline`` times the CPU oracle (the
reference's gather-then-dense PyTorch path, restated in oracle/) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO / "mini-vllm_amd", REPO):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

METRIC = "paged-attn decode HBM GB/s (% of peak) + engine decode tok/s, Qwen3-0.6B"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def measured_traffic() -> int | None:
    """HBM bytes per decode launch from the committed counter summary (two rocprofv3
    --pmc passes, calibrated on a copy of known size), or None if there is none."""
    path = REPO / "profiles" / "paged_decode_cfg2_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_steps(fn, steps: int, warmup: int) -> float:
    """Mean ms per call over `steps` back-to-back calls.

    Two HIP events on the stream the kernels run on bracket the whole loop; no event
    is recorded between calls, because a timed event record makes the GPU drain and
    flush the previous kernel before dispatching the next one, which would add a gap
    to every step that a real decode loop does not have.
    """
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    first = torch.cuda.Event(enable_timing=True)
    last = torch.cuda.Event(enable_timing=True)
    first.record(stream)
    for i in range(steps):
        fn(i)
    last.record(stream)
    torch.cuda.synchronize()
    return first.elapsed_time(last) / steps


def rotated_batches(index: int, copies: int, kv_dtype=None):
    """`copies` batches sharing shapes and tables, each with its own K/V pools."""
    from mini_vllm.workloads import config_batch

    base = config_batch(index, device="cuda", generator_device="cuda", kv_dtype=kv_dtype)
    batches = [base]
    for c in range(1, copies):
        other = config_batch(index, device="cuda", seed=0, generator_device="cuda", kv_dtype=kv_dtype)
        gen = torch.Generator(device="cuda").manual_seed(1000 + c)
        if other.key_pool.dtype == torch.float8_e4m3fn:
            # fresh fp8 codes with the same scales: any finite code pattern is valid data
            other.key_pool = torch.randint(0, 126, other.key_pool.shape, generator=gen,
                                           device="cuda", dtype=torch.uint8).view(torch.float8_e4m3fn)
            other.value_pool = torch.randint(0, 126, other.value_pool.shape, generator=gen,
                                             device="cuda", dtype=torch.uint8).view(torch.float8_e4m3fn)
        else:
            other.key_pool = torch.randn(other.key_pool.shape, generator=gen, device="cuda").to(other.key_pool.dtype)
            other.value_pool = torch.randn(other.value_pool.shape, generator=gen, device="cuda").to(other.value_pool.dtype)
        batches.append(other)
    return batches


def run_paged(batches, steps, warmup):
    from mini_vllm.kernels import ops

    def step(i):
        b = batches[i % len(batches)]
        ops.paged_attention(*b.args(), use_cuda=True, k_scale=b.k_scale, v_scale=b.v_scale)

    return time_steps(step, steps, warmup)


def run_engine(requests: int = 256, max_tokens: int = 256, max_sequences: int = 32,
               use_graphs: bool = True, kv_dtype: torch.dtype | None = None) -> dict:
    """a Qwen3-0.6B-shaped model (random init, std 0.02, bf16) served
    by the paged engine with the HIP kernels: `requests` prompts of U[64, 2048] random
    token ids (seed 0), `max_tokens` greedy tokens each (EOS ignored), continuous
    batching with a 2048-token budget, 512-token chunks, `max_sequences` in flight."""
    from mini_vllm.block import BlockManager
    from mini_vllm.model import ModelConfig, Qwen3Paged, random_weights
    from mini_vllm.serve import LLMEngine, SchedulerConfig
    from mini_vllm.workloads import (CONFIG5_BUDGET, CONFIG5_CHUNK, config5_pool_blocks,
                                     config5_prompts)

    config = ModelConfig()
    weights = random_weights(config, seed=0, device="cuda")
    prompts = config5_prompts(requests, config.vocab_size)
    lens = [len(p) for p in prompts]
    blocks = config5_pool_blocks(max_sequences, max_tokens)
    sched = SchedulerConfig(max_batched_tokens=CONFIG5_BUDGET, max_sequences=max_sequences,
                            chunk_size=CONFIG5_CHUNK)

    def engine():
        manager = BlockManager(blocks, 16, config.num_hidden_layers, config.num_key_value_heads,
                               config.head_dim, kv_dtype or config.dtype, "cuda")
        return LLMEngine(Qwen3Paged(config, weights, manager, use_cuda=True), sched, device="cuda",
                         use_graphs=use_graphs)

    warm = engine()
    warm.generate(prompts[:4], 4)  # warm up kernels and BLAS handles
    # the hipBLASLt entry chooses its algorithm per row-count class at first use: do it
    # for every class the 2048-token budget can produce before the timed run
    tuned = warm.model.prepare_prefill_products(CONFIG5_BUDGET)
    del warm
    torch.cuda.synchronize()
    eng = engine()
    eng.generate(prompts, max_tokens)
    torch.cuda.synchronize()
    st = eng.stats
    return {
        "requests": requests, "max_tokens": max_tokens, "max_sequences": max_sequences,
        "prompt_tokens": sum(lens), "generated_tokens": st.generated_tokens,
        "iterations": st.iterations, "preemptions": st.preemptions,
        "elapsed_s": round(st.elapsed_s, 3),
        "output_tok_s": round(st.output_tokens_per_s, 1),
        "decode_tok_s": round(st.decode_tokens_per_s, 1),
        "decode_only_iterations": st.decode_only_iterations,
        "decode_graphs": use_graphs,
        "kv_dtype": str(kv_dtype or config.dtype).replace("torch.", ""),
        "prefill_products_prepared": tuned,
    }


def run_decode_step(steps: int = 40, warmup: int = 8, batch: int = 32, context: int = 1024) -> dict:
    """One decode iteration of config 5's engine at a fixed shape: `batch` sequences whose
    prompts (`context` random ids, seed 0) were prefilled by the engine, then `steps`
    pure-decode iterations (the decode graphs, greedy, EOS ignored) timed back to back
    with the host scheduling each next one while the GPU runs the current (what config 5
    runs 92% of the time). Algorithmic bytes per step: every weight the forward reads
    once (28 layers of q/k/v, o, gate/up, down; the LM head; norm weights) plus each
    sequence's K and V over its context at that step, 2 bytes an element."""
    from mini_vllm.block import BlockManager
    from mini_vllm.model import ModelConfig, Qwen3Paged, random_weights
    from mini_vllm.serve import LLMEngine, SchedulerConfig
    from mini_vllm.workloads import CONFIG5_BUDGET, CONFIG5_CHUNK

    config = ModelConfig()
    weights = random_weights(config, seed=0, device="cuda")
    gen = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, config.vocab_size, (context,), generator=gen).tolist()
               for _ in range(batch)]
    total_tokens = context + warmup + steps + 4
    blocks = batch * (-(-total_tokens // 16)) + 64
    sched = SchedulerConfig(max_batched_tokens=CONFIG5_BUDGET, max_sequences=batch,
                            chunk_size=CONFIG5_CHUNK)
    manager = BlockManager(blocks, 16, config.num_hidden_layers, config.num_key_value_heads,
                           config.head_dim, config.dtype, "cuda")
    eng = LLMEngine(Qwen3Paged(config, weights, manager, use_cuda=True), sched, device="cuda",
                    use_graphs=True)
    seqs = [eng.add_request(p, warmup + steps + 4) for p in prompts]
    while any(len(s.output) == 0 for s in seqs):  # prefill (and the first token)
        eng.step()
    for _ in range(warmup):
        eng.step()
    torch.cuda.synchronize()
    ctx0 = min(len(s) for s in seqs)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.step(resolve_finished=False)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    eng.flush()
    c, layers = config, config.num_hidden_layers
    per_layer = (c.q_size + 2 * c.kv_size) * c.hidden_size + c.hidden_size * c.q_size + \
        2 * c.intermediate_size * c.hidden_size + c.hidden_size * c.intermediate_size
    weight_bytes = 2 * (layers * per_layer + c.vocab_size * c.hidden_size)
    mean_ctx = ctx0 + (steps - 1) / 2.0
    kv_bytes = 2 * 2 * batch * mean_ctx * layers * c.num_key_value_heads * c.head_dim
    gbs = (weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9
    return {"batch": batch, "context_at_start": ctx0, "steps": steps, "ms_per_step": round(ms, 4),
            "output_tok_s": round(batch / (ms * 1e-3), 1),
            "weight_bytes": int(weight_bytes), "kv_bytes_mean": int(kv_bytes),
            "gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / 8000.0, 4)}


def run_prefill_occupancy(steps: int = 20, tiles: int = 16) -> dict:
    """Items of `tiles` 64-key tiles (128 queries after a prefix, bf16, GQA 16/8, D 128) on
    the item grid, as many as half the CUs and as all of them: the per-tile cost of one
    CU when every CU is busy against when half are (a counter pass under rocprofv3 tells
    the two launches apart by their grid size)."""
    from mini_vllm.kernels import ops  # noqa: F401  (strict-mode import side effects)
    from mini_vllm.kernels.extension import load_extension
    from mini_vllm.workloads import build_batch

    ext = load_extension()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = {}
    for items in (cus // 2, cus):
        seqs = items // 8
        b = build_batch([64 * tiles] * seqs, [128] * seqs, dtype=torch.bfloat16,
                        num_q_heads=16, num_kv_heads=8, head_dim=128, seed=0, device="cuda",
                        generator_device="cuda")
        opts = {"prefill_schedule": "grid", "prefill_pieces": 1}
        ms = time_steps(lambda i: ext.paged_attention(*b.args(), plan_options=opts), steps, 3)
        out[f"items{items}"] = {"us": round(ms * 1e3, 1), "us_per_tile": round(ms * 1e3 / tiles, 2)}
        del b
    return out


def run_kv_write(steps: int = 20) -> dict:
    """The paged KV write (one layer, 8 kv heads x 128, 16-token pages): 2048 tokens (one
    engine iteration's budget) and 65536 tokens (bandwidth), into shuffled slots of a
    pool with 10% spare pages. Bytes = K and V read from the token rows + written to the
    pool (bf16), or read (bf16) + written (fp8) + scales."""
    from mini_vllm.kernels import ops

    out = {}
    hk, d, bs = 8, 128, 16
    for tokens in (2048, 65536):
        pages = -(-tokens // bs)
        nb = int(pages * 1.1) + 1
        gen = torch.Generator().manual_seed(tokens)
        perm = torch.randperm(nb, generator=gen)[:pages]
        slots = (perm[:, None] * bs + torch.arange(bs)).reshape(-1)[:tokens].to(torch.int32).cuda()
        key = torch.randn(tokens, hk, d, device="cuda", dtype=torch.bfloat16)
        value = torch.randn(tokens, hk, d, device="cuda", dtype=torch.bfloat16)
        for kv in (torch.bfloat16, torch.float8_e4m3fn):
            kp = torch.zeros(nb, bs, hk, d, device="cuda", dtype=kv)
            vp = torch.zeros_like(kp)
            sc = {}
            if kv == torch.float8_e4m3fn:
                sc = dict(k_scale=torch.zeros(nb, hk, device="cuda"),
                          v_scale=torch.zeros(nb, hk, device="cuda"))
            ms = time_steps(lambda i: ops.kv_write(kp, vp, key, value, slots, use_cuda=True, **sc),
                            steps, 3)
            elt = kp.element_size()
            nbytes = 2 * tokens * hk * d * (2 + elt) + (2 * pages * hk * 4 * 2 if sc else 0)
            name = f"T{tokens}_{'fp8' if sc else 'bf16'}"
            out[name] = {"us": round(ms * 1e3, 1), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
            log(f"kv_write {name}: {ms * 1e3:.1f} us, {out[name]['gbs']:.0f} GB/s")
    return out


def run_dense(steps: int = 20) -> dict:
    """Dense-cache attention (``ops.attention``, reference csrc/decode_attention.cu and
    csrc/flash_prefill.cu) on the paged kernels, against the PyTorch path on the same
    GPU: decode B=32 x S=2048 read in place from a cache preallocated for 4096 positions
    (bytes = K + V read once), and causal prefill B=8 x L=512 after a 512-token prefix
    (FLOPs over visible pairs), bf16, 16q/8kv heads, D=128."""
    from mini_vllm.kernels import ops

    bf = torch.bfloat16
    out = {}
    b, hq, hk, d = 32, 16, 8, 128
    S, s_max = 2048, 4096
    caches = [(torch.randn(b, hk, s_max, d, device="cuda", dtype=bf)[:, :, :S],
               torch.randn(b, hk, s_max, d, device="cuda", dtype=bf)[:, :, :S]) for _ in range(3)]
    q = torch.randn(b, hq, 1, d, device="cuda", dtype=bf)
    nbytes = 2 * b * hk * S * d * 2
    for name, use in (("kernel", True), ("torch", False)):
        ms = time_steps(lambda i: ops.attention(q, *caches[i % 3], use_cuda=use), steps, 3)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"decode_{name}"] = {"us": round(ms * 1e3, 1), "gbs": round(gbs, 1)}
        log(f"dense decode ({name}): {ms * 1e3:.1f} us, {gbs:.0f} GB/s")
    del caches
    b, L, S = 8, 512, 1024
    qs = [torch.randn(b, hq, L, d, device="cuda", dtype=bf) for _ in range(3)]
    kv = [(torch.randn(b, hk, S, d, device="cuda", dtype=bf),
           torch.randn(b, hk, S, d, device="cuda", dtype=bf)) for _ in range(3)]
    flops = 4 * hq * d * b * (L * (S - L) + L * (L + 1) // 2)
    for name, use in (("kernel", True), ("torch", False)):
        ms = time_steps(lambda i: ops.attention(qs[i % 3], *kv[i % 3], mask="causal", use_cuda=use),
                        steps, 3)
        tf = flops / (ms * 1e-3) / 1e12
        out[f"prefill_{name}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1)}
        log(f"dense prefill ({name}): {ms * 1e3:.1f} us, {tf:.0f} TFLOP/s")
    del qs, kv
    torch.cuda.empty_cache()
    return out


def graph_time(fn, calls: int, replays: int = 5) -> float:
    """Mean ms per call of ``fn(0) .. fn(calls - 1)`` captured in one HIP graph and
    replayed: the GPU-side cost of a launch-sized op without the Python between calls
    (what a captured decode step sees)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(calls):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(calls):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    first = torch.cuda.Event(enable_timing=True)
    last = torch.cuda.Event(enable_timing=True)
    first.record()
    for _ in range(replays):
        graph.replay()
    last.record()
    torch.cuda.synchronize()
    del graph
    return first.elapsed_time(last) / (replays * calls)


def run_linear(steps: int = 20) -> dict:
    """The decode step's projections (Qwen3-0.6B shapes, 32 rows = config 5's running
    sequences, bf16) on the skinny kernels over packed weights against torch's BLAS on
    the row-major ones, each call reading a different weight copy (> 1 GB rotated, so
    the weights come from HBM as in a decode iteration). Bytes = weights + x + y. Timed
    as replays of a captured graph of back-to-back calls (``graph_time``), as the decode
    step runs them; the Python of an eager call costs more than these kernels."""
    from mini_vllm import torch_path
    from mini_vllm.kernels import ops

    bf = torch.bfloat16
    m = 32
    shapes = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up_swiglu": (6144, 1024),
              "down": (1024, 3072), "lm_head": (151936, 1024)}
    out = {}
    for name, (n, k) in shapes.items():
        copies = max(3, int(1.2e9 // (n * k * 2)))
        dense = [torch.randn(n, k, device="cuda", dtype=bf) * 0.02 for _ in range(copies)]
        if name == "gate_up_swiglu":
            dense = [torch_path.interleave_gate_up(w[: n // 2], w[n // 2:]) for w in dense]
        packed = [ops.pack_weight(w, use_cuda=True) for w in dense]
        x = torch.randn(m, k, device="cuda", dtype=bf)
        r = torch.randn(m, n, device="cuda", dtype=bf)
        if name == "qkv":
            call = lambda i: ops.linear_split(x, packed[i % copies], (2048, 1024, 1024), use_cuda=True)
        elif name in ("o", "down"):
            call = lambda i: ops.linear_residual(x, packed[i % copies], r, use_cuda=True)
        elif name == "gate_up_swiglu":
            call = lambda i: ops.linear_swiglu(x, packed[i % copies], use_cuda=True)
        else:
            call = lambda i: ops.linear(x, packed[i % copies], use_cuda=True)
        nbytes = 2 * n * k + 2 * m * k + 2 * m * n
        ms = graph_time(call, min(steps, copies))
        blas_ms = graph_time(lambda i: x @ dense[i % copies].t(), min(steps, copies))
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"n": n, "k": k, "us": round(ms * 1e3, 1), "gbs": round(gbs, 1),
                     "blas_us": round(blas_ms * 1e3, 1)}
        log(f"linear {name} ({m}x{n}x{k}): {ms * 1e3:.1f} us, {gbs:.0f} GB/s; BLAS {blas_ms * 1e3:.1f} us")
        del dense, packed
        torch.cuda.empty_cache()
    logits = [torch.randn(m, 151936, device="cuda", dtype=bf) for _ in range(3)]
    ms = graph_time(lambda i: ops.argmax(logits[i % 3], use_cuda=True), steps)
    torch_ms = graph_time(lambda i: logits[i % 3].argmax(dim=-1), steps)
    out["argmax_32x151936"] = {"us": round(ms * 1e3, 1), "torch_us": round(torch_ms * 1e3, 1)}
    log(f"argmax 32x151936: {ms * 1e3:.1f} us; torch {torch_ms * 1e3:.1f} us")
    return out


def run_prefill_gemm(steps: int = 20, tokens: int = 2048) -> dict:
    """The four projections of a config-5 prefill iteration (2048 tokens, Qwen3-0.6B
    shapes, bf16, fp32 accumulate) as the model runs them (``ops.linear``: the library's
    hipBLASLt entry, whose first call of a shape times the heuristic's 16 candidates and
    keeps the fastest; then again after ``blas_tune`` has swept every algorithm for the
    shape, as the engine's start-up does), against torch's product (the same library,
    the heuristic's first algorithm, set-up made per call). Four weight copies rotated;
    timed as graph replays of back-to-back calls. FLOPs = 2 M N K. ``choice`` is the
    library's record of how it chose (candidates, the kept one's index - past 15 one of
    the sweep's - and the heuristic first's and the kept one's time)."""
    from mini_vllm.kernels import ops
    from mini_vllm.kernels.extension import load_extension

    ext = load_extension()
    bf = torch.bfloat16
    shapes = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072)}
    out = {}
    for name, (n, k) in shapes.items():
        ws = [torch.randn(n, k, device="cuda", dtype=bf) * 0.02 for _ in range(4)]
        x = torch.randn(tokens, k, device="cuda", dtype=bf)
        flop = 2 * tokens * n * k
        def rounded(choice):
            return {key: round(v, 2) if isinstance(v, float) else v for key, v in choice.items()}

        blas_ms = graph_time(lambda i: x @ ws[i % 4].t(), steps)
        # the heuristic's first 16 algorithms, timed at the first call
        h_ms = graph_time(lambda i: ops.linear(x, ws[i % 4], use_cuda=True), steps)
        h_choice = ext.blas_choice(tokens, n, k, bf)
        # with every algorithm swept once (as prepare_prefill_products does at start-up)
        swept = ext.blas_tune(x, ws[0])
        ms = graph_time(lambda i: ops.linear(x, ws[i % 4], use_cuda=True), steps)
        choice = ext.blas_choice(tokens, n, k, bf)
        tflops = flop / (ms * 1e-3) / 1e12
        out[name] = {"m": tokens, "n": n, "k": k, "us": round(ms * 1e3, 1),
                     "tflops": round(tflops, 1),
                     "frac_of_bf16_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4),
                     "algorithms_swept": swept, "choice": rounded(choice),
                     "heuristic_us": round(h_ms * 1e3, 1), "heuristic_choice": rounded(h_choice),
                     "torch_us": round(blas_ms * 1e3, 1),
                     "torch_tflops": round(flop / (blas_ms * 1e-3) / 1e12, 1)}
        log(f"prefill projection {name} ({tokens}x{n}x{k}): {ms * 1e3:.1f} us, {tflops:.0f} "
            f"TFLOP/s after sweeping {swept} algorithms (heuristic's 16: {h_ms * 1e3:.1f} us; "
            f"torch {blas_ms * 1e3:.1f} us); choice {choice}")
        del ws
        torch.cuda.empty_cache()
    return out


def run_elementwise(steps: int = 20) -> dict:
    """RMSNorm (E=1024 and per-head D=128), RoPE (16 heads x 128) and SwiGLU (I=3072)
    at bf16 on ~256 MB operands, three rotated copies each so every call reads HBM.
    Bytes are algorithmic (the reference's rule, mini_vllm/bench.py:531-580): inputs
    read once and outputs written once; RoPE also reads each token's cos/sin rows."""
    from mini_vllm.kernels import ops
    from mini_vllm.torch_path import rope_tables

    bf = torch.bfloat16
    out = {}

    def measure(name, make, call, nbytes):
        bufs = [make() for _ in range(3)]
        ms = time_steps(lambda i: call(*bufs[i % 3]), steps, 3)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 1), "gbs": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"elementwise {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s")
        del bufs
        torch.cuda.empty_cache()

    rows = 1 << 17
    w = torch.ones(1024, device="cuda", dtype=bf)
    measure("rmsnorm_E1024", lambda: (torch.randn(rows, 1024, device="cuda", dtype=bf),),
            lambda x: ops.rmsnorm(x, w, 1e-6, use_cuda=True), 2 * rows * 1024 * 2 + 1024 * 2)
    wq = torch.ones(128, device="cuda", dtype=bf)
    tokens = 1 << 16
    measure("qk_norm_16x128", lambda: (torch.randn(tokens, 16, 128, device="cuda", dtype=bf),),
            lambda x: ops.rmsnorm(x, wq, 1e-6, use_cuda=True), 2 * tokens * 16 * 128 * 2 + 256)
    cos, sin = rope_tables(128, tokens, device="cuda")
    pos = torch.arange(tokens, device="cuda")
    measure("rope_16x128", lambda: (torch.randn(1, tokens, 16, 128, device="cuda", dtype=bf),),
            lambda x: ops.rope(x, pos, cos, sin, use_cuda=True),
            2 * tokens * 16 * 128 * 2 + 2 * tokens * 128 * 4)
    wk = torch.ones(128, device="cuda", dtype=bf)
    measure("qk_norm_rope_16q8k_x128",
            lambda: (torch.randn(tokens, 16, 128, device="cuda", dtype=bf),
                     torch.randn(tokens, 8, 128, device="cuda", dtype=bf)),
            lambda q, k: ops.qk_norm_rope(q, k, wq, wk, pos, cos, sin, 1e-6, use_cuda=True),
            2 * tokens * 24 * 128 * 2 + 2 * tokens * 128 * 4 + 512)
    measure("swiglu_I3072", lambda: (torch.randn(tokens, 3072, device="cuda", dtype=bf),
                                     torch.randn(tokens, 3072, device="cuda", dtype=bf)),
            lambda g, u: ops.swiglu(g, u, use_cuda=True), 3 * tokens * 3072 * 2)
    return out


class ClockSampler:
    """Polls ``amd-smi metric --clock`` in a background thread and keeps the highest
    graphics clock (the busiest XCD) and memory clock seen, as the reference's
    ClockSampler does with nvidia-smi (mini_vllm/bench.py:113-235): one reading taken
    after the work has finished shows idle clocks, the peak over the run shows whether
    the card was allowed to run fast while it was measured. A run whose peak is below
    half the maximum graphics or memory clock is flagged as throttled (the reference's
    threshold, :135-143)."""

    def __init__(self, interval: float = 1.0) -> None:
        import shutil
        import threading

        self.interval = interval
        self.available = shutil.which("amd-smi") is not None
        self.samples = 0
        self.peak_gfx = self.max_gfx = self.peak_mem = self.max_mem = 0
        self.first = self.last = None
        self.loaded = None
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._poll, daemon=True) if self.available else None

    @staticmethod
    def read() -> dict | None:
        import subprocess

        try:
            out = subprocess.run(["amd-smi", "metric", "-g", "0", "--clock", "--json"],
                                 capture_output=True, text=True, timeout=10, check=True).stdout
            data = json.loads(out)
            clocks = (data["gpu_data"] if isinstance(data, dict) else data)[0]["clock"]
        except (subprocess.SubprocessError, OSError, ValueError, KeyError, IndexError, TypeError):
            return None

        def mhz(entry, key):
            v = entry.get(key) if isinstance(entry, dict) else None
            return int(v["value"]) if isinstance(v, dict) and "value" in v else 0

        gfx = [c for k, c in clocks.items() if k.startswith("gfx")]
        mem = [c for k, c in clocks.items() if k.startswith("mem")]
        return {"gfx_mhz": max((mhz(c, "clk") for c in gfx), default=0),
                "gfx_max_mhz": max((mhz(c, "max_clk") for c in gfx), default=0),
                "mem_mhz": max((mhz(c, "clk") for c in mem), default=0),
                "mem_max_mhz": max((mhz(c, "max_clk") for c in mem), default=0)}

    def _poll(self) -> None:
        while not self._stop.is_set():
            r = self.read()
            if r is not None:
                self.samples += 1
                self.first = self.first or r
                self.last = r
                self.peak_gfx = max(self.peak_gfx, r["gfx_mhz"])
                self.peak_mem = max(self.peak_mem, r["mem_mhz"])
                self.max_gfx = max(self.max_gfx, r["gfx_max_mhz"])
                self.max_mem = max(self.max_mem, r["mem_max_mhz"])
            self._stop.wait(self.interval)

    def __enter__(self) -> "ClockSampler":
        if self._thread is not None:
            self._thread.start()
        return self

    def __exit__(self, *exc) -> None:
        self._stop.set()
        if self._thread is not None:
            self._thread.join(timeout=15)

    def under_load(self, fn, step_ms: float, seconds: float = 1.5) -> dict | None:
        """One reading taken while the GPU runs ``fn(i)`` back to back: enough calls are
        enqueued for ``seconds`` of GPU work, the clocks are read while they run, then
        the stream is drained. A short timed region (config 2's 50 steps take ~6 ms)
        is over long before one amd-smi call returns, so this is the reading that says
        what the clocks are while the headline workload runs."""
        if not self.available:
            return None
        n = max(1, int(seconds * 1e3 / max(step_ms, 1e-3)))
        torch.cuda.synchronize()
        for i in range(n):
            fn(i)
        r = self.read()
        torch.cuda.synchronize()
        if r is not None:
            self.loaded = r
            self.peak_gfx = max(self.peak_gfx, r["gfx_mhz"])
            self.peak_mem = max(self.peak_mem, r["mem_mhz"])
            self.max_gfx = max(self.max_gfx, r["gfx_max_mhz"])
            self.max_mem = max(self.max_mem, r["mem_max_mhz"])
        return r

    def report(self) -> dict:
        loaded = self.loaded
        if not self.available or (self.samples == 0 and loaded is None):
            return {"available": False, "reason": "amd-smi missing or unreadable"}
        # judged on the reading under the headline load when there is one (a background
        # sample may fall between GPU legs, at idle clocks), else the peak over the run
        gfx = loaded["gfx_mhz"] if loaded else self.peak_gfx
        mem = loaded["mem_mhz"] if loaded else self.peak_mem
        throttled = (self.max_gfx and gfx < 0.5 * self.max_gfx) or \
            (self.max_mem and mem < 0.5 * self.max_mem)
        return {"available": True, "samples": self.samples, "interval_s": self.interval,
                "under_headline_load": loaded,
                "peak_gfx_mhz": self.peak_gfx, "max_gfx_mhz": self.max_gfx,
                "peak_mem_mhz": self.peak_mem, "max_mem_mhz": self.max_mem,
                "first_sample": self.first, "last_sample": self.last,
                "throttled": bool(throttled)}


def read_ceiling(steps: int = 20, total_bytes: int = 2 << 30, page_bytes: int = 32768) -> dict:
    """Read-only HBM ceilings from the library's probe (``mvllm_read_probe``): a 2 GiB
    buffer (8x the Infinity Cache) read as 32 KB pages - one paged pool's page of 16
    rows x 8 kv heads x 128 bf16 - in address order and in a shuffled order (as the
    decode reads its pages), each at several resident workgroup counts, best of them.
    The paged decode's own rate is bounded by the shuffled figure; a device copy (the
    reference's ceiling) moves reads and writes at once and lands below the decode."""
    from mini_vllm.kernels.extension import load_extension

    ext = load_extension()
    base = torch.empty(total_bytes, dtype=torch.uint8, device="cuda")
    base.view(torch.int32).random_()
    pages = total_bytes // page_bytes
    gen = torch.Generator().manual_seed(0)
    shuffled = torch.randperm(pages, generator=gen).to(torch.int32).cuda()
    out = {"buffer_bytes": total_bytes, "page_bytes": page_bytes}
    for name, ids in (("sequential", None), ("shuffled_pages", shuffled)):
        best = (0.0, 0)
        for wgs in (256, 512, 1024, 2048):
            sink = torch.empty(wgs * 256, dtype=torch.int32, device="cuda")
            ms = time_steps(lambda i: ext.read_probe(base, page_bytes, ids, wgs, sink), steps, 3)
            gbs = total_bytes / (ms * 1e-3) / 1e9
            best = max(best, (gbs, wgs))
        out[f"{name}_gbs"] = round(best[0], 1)
        out[f"{name}_workgroups"] = best[1]
        log(f"read ceiling {name}: {best[0]:.0f} GB/s ({best[1]} workgroups)")
    del base, shuffled
    torch.cuda.empty_cache()
    return out


def run_kernel_cases(steps: int = 20) -> dict:
    """The reference's own kernel-benchmark shapes (mini_vllm/bench.py:617-691, bf16,
    16q/8kv heads, D 128, 16-token pages, shuffled tables): paged decode at (B, S) in
    {(1, 8192), (16, 1024), (64, 1024)} - bytes = 2 B S H_k D x 2, the reference's rule
    (:643) - and a prefill chunk at (L, S) in {(512, 2048), (2048, 2048)} - FLOPs over
    visible pairs, and the reference's bytes moved (q + K + V). Decode pools are rotated
    over enough copies that a step's pages are not in the 256 MB Infinity Cache. Each
    against the PyTorch path (the reference's gather-then-dense oracle) on the same GPU,
    the speedup column of the reference's table."""
    from mini_vllm.kernels import ops
    from mini_vllm.workloads import build_batch, prefill_flops

    out = {}
    for b, S in ((1, 8192), (16, 1024), (64, 1024)):
        kv = 2 * b * S * 8 * 128 * 2
        copies = max(2, -(-600_000_000 // kv))
        batches = [build_batch([S] * b, [1] * b, dtype=torch.bfloat16, seed=c, spare_blocks=0,
                               device="cuda", generator_device="cuda") for c in range(copies)]
        ms = run_paged(batches, steps, 3)
        torch_ms = time_steps(lambda i: ops.paged_attention(*batches[i % copies].args(),
                                                            use_cuda=False), 3, 1)
        gbs = kv / (ms * 1e-3) / 1e9
        out[f"decode_B{b}_S{S}"] = {"us": round(ms * 1e3, 1), "kv_bytes": kv,
                                    "gbs": round(gbs, 1),
                                    "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                    "rotated_copies": copies, "torch_path_us": round(torch_ms * 1e3, 1),
                                    "speedup_vs_torch_path": round(torch_ms / ms, 1)}
        log(f"kernel case decode B={b} S={S}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s; "
            f"torch path {torch_ms * 1e3:.0f} us ({torch_ms / ms:.0f}x)")
        del batches
    for L, S in ((512, 2048), (2048, 2048)):
        batches = [build_batch([S], [L], dtype=torch.bfloat16, seed=c, spare_blocks=0,
                               device="cuda", generator_device="cuda") for c in range(2)]
        ms = run_paged(batches, steps, 3)
        torch_ms = time_steps(lambda i: ops.paged_attention(*batches[i % 2].args(), use_cuda=False),
                              3, 1)
        flops = prefill_flops(batches[0])
        moved = (batches[0].q.numel() + 2 * S * 8 * 128) * 2
        tflops = flops / (ms * 1e-3) / 1e12
        out[f"prefill_L{L}_S{S}"] = {"us": round(ms * 1e3, 1), "gflop": round(flops / 1e9, 3),
                                     "tflops": round(tflops, 1),
                                     "frac_of_bf16_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4),
                                     "bytes_moved": moved,
                                     "torch_path_us": round(torch_ms * 1e3, 1),
                                     "speedup_vs_torch_path": round(torch_ms / ms, 1)}
        log(f"kernel case prefill L={L} S={S}: {ms * 1e3:.1f} us, {tflops:.0f} TFLOP/s; "
            f"torch path {torch_ms * 1e3:.0f} us ({torch_ms / ms:.0f}x)")
        del batches
    torch.cuda.empty_cache()
    return out


def copy_ceiling(nbytes: int, steps: int = 20) -> float:
    """GB/s of a device-to-device copy_ (read + write counted), the practical ceiling
    (method of the reference's mini_vllm/bench.py:448-466)."""
    n = nbytes // 2
    src = [torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(2)]
    dst = [torch.empty_like(s) for s in src]

    def step(i):
        dst[i % 2].copy_(src[i % 2])

    ms = time_steps(step, steps, 3)
    return 2 * n * 2 / (ms * 1e-3) / 1e9


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _sub_batch(b, seqs: list[int]):
    """The rows of sequences ``seqs`` of a PagedBatch (same pools), for a bounded CPU
    sample: sequences are independent, so a subset is the same work per sequence."""
    from mini_vllm.workloads import PagedBatch

    cu = [int(v) for v in b.cu_seqlens_q]
    rows = torch.cat([torch.arange(cu[s], cu[s + 1]) for s in seqs])
    lens = [cu[s + 1] - cu[s] for s in seqs]
    new_cu = torch.tensor([0] + lens, dtype=torch.int32).cumsum(0, dtype=torch.int32)
    return PagedBatch(b.q[rows], b.key_pool, b.value_pool, b.block_tables[seqs].contiguous(), new_cu,
                      b.context_lens[seqs], b.seq_lens[seqs], max(lens),
                      max(b.contexts[s] for s in seqs), b.scale, b.k_scale, b.v_scale,
                      [b.contexts[s] for s in seqs], lens)


def _median_time(fn, runs: int = 5) -> tuple[float, int]:
    fn()  # warmup
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline() -> dict:
    """The reference's CPU path (its gather-then-dense PyTorch attention,
    ``ops.paged_attention(use_cuda=False)``, mini_vllm/paged_attention.py:36-110) on the
    host cores, for BASELINE configs 1-4 in their own dtype and in fp32 (median of 5 runs
    after a warmup, on the same seeded inputs; configs 2 and 4 on a stated sample of
    their sequences), and a stated subset of config 5 through the engine with the
    kernels off. The headline entry is config 2 in bf16; ``configs`` holds the rest."""
    from mini_vllm.kernels import ops
    from mini_vllm.workloads import config_batch, prefill_flops

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    configs = {}

    def attention_leg(name, b, work, unit, sample):
        for leg in ("native", "fp32") if b.q.dtype != torch.float32 else ("native",):
            q = b.q if leg == "native" else b.q.float()
            fp8 = b.key_pool.dtype == torch.float8_e4m3fn
            kp = b.key_pool if leg == "native" or fp8 else b.key_pool.float()
            vp = b.value_pool if leg == "native" or fp8 else b.value_pool.float()
            args = (q, kp, vp, b.block_tables, b.cu_seqlens_q, b.context_lens, b.seq_lens,
                    b.max_query_len, b.max_context_len, b.scale)
            med, runs = _median_time(lambda: ops.paged_attention(
                *args, use_cuda=False, k_scale=b.k_scale, v_scale=b.v_scale))
            dtype = str(q.dtype).replace("torch.", "")
            configs[f"{name}_{dtype}"] = {
                "value": round(work / med / (1e9 if unit == "GB/s" else 1e12), 4), "unit": unit,
                "ms": round(med * 1e3, 2), "runs": runs, "sample": sample}
            log(f"cpu {name} {dtype}: {med * 1e3:.1f} ms, {configs[f'{name}_{dtype}']['value']} {unit}")

    b1 = config_batch(1)
    attention_leg("config1", b1, b1.kv_bytes(), "GB/s", "all 4 sequences (fp32 inputs)")
    b2 = config_batch(2)
    s2 = _sub_batch(b2, list(range(8)))
    attention_leg("config2", s2, s2.kv_bytes(), "GB/s",
                  f"sequences 0-7 of 64 (ctx {s2.contexts})")
    b3 = config_batch(3)
    attention_leg("config3", b3, prefill_flops(b3), "TFLOP/s", "all 8 sequences x 512 queries")
    b4 = config_batch(4)
    s4 = _sub_batch(b4, list(range(4)))
    attention_leg("config4", s4, s4.kv_bytes() + s4.scale_bytes(), "GB/s",
                  f"sequences 0-3 of 128 (ctx {s4.contexts}), fp8 pool dequantised")
    del b2, b3, b4
    configs["config5_subset"] = _cpu_engine_subset()

    head = configs["config2_bfloat16"]
    return {
        "value": head["value"],
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"config 2 in bf16: {head['sample']}; ops.paged_attention(use_cuda=False), the "
                  f"reference's gather-then-dense path; median of {head['runs']} runs, {head['ms']} ms",
        "cpu_model": _cpu_model(),
        "configs": configs,
    }


def _cpu_engine_subset(requests: int = 8, prompt_tokens: int = 128, max_tokens: int = 32) -> dict:
    """Config 5 on the host cores, kernels off: the first ``requests`` config-5 prompts
    trimmed to ``prompt_tokens`` tokens, ``max_tokens`` greedy tokens each, through the
    same engine (bf16 Qwen3-0.6B shape, random init seed 0, 2048-token budget, 512-token
    chunks). A subset: the whole workload would take hours on a CPU."""
    from mini_vllm.block import BlockManager
    from mini_vllm.model import ModelConfig, Qwen3Paged, random_weights
    from mini_vllm.serve import LLMEngine, SchedulerConfig
    from mini_vllm.workloads import CONFIG5_BUDGET, CONFIG5_CHUNK, config5_prompts

    config = ModelConfig()
    weights = random_weights(config, seed=0)
    prompts = [p[:prompt_tokens] for p in config5_prompts(requests, config.vocab_size)]
    blocks = requests * -(-(prompt_tokens + max_tokens) // 16) + 1
    manager = BlockManager(blocks, 16, config.num_hidden_layers, config.num_key_value_heads,
                           config.head_dim, config.dtype, "cpu")
    engine = LLMEngine(Qwen3Paged(config, weights, manager, use_cuda=False),
                       SchedulerConfig(max_batched_tokens=CONFIG5_BUDGET, chunk_size=CONFIG5_CHUNK))
    engine.generate(prompts, max_tokens)
    st = engine.stats
    log(f"cpu config 5 subset: {st.output_tokens_per_s:.1f} output tok/s")
    return {"value": round(st.output_tokens_per_s, 2), "unit": "output tok/s",
            "decode_tok_s": round(st.decode_tokens_per_s, 2), "elapsed_s": round(st.elapsed_s, 2),
            "sample": f"{requests} requests: config-5 prompts 0-{requests - 1} trimmed to "
                      f"{prompt_tokens} tokens, {max_tokens} greedy tokens each, bf16, "
                      "use_cuda=False (one run)"}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--copies", type=int, default=3, help="rotated pool copies (defeat the MALL)")
    parser.add_argument("--skip-extras", action="store_true", help="headline config 2 only")
    parser.add_argument("--extras", default="3,3fp8,4,5,step,ew,kv,dense,linear,gemm,ceiling,cases",
                        help="comma list of extras to run: 3 (prefill), 3fp8 (prefill over an "
                             "fp8 pool), 4 (fp8 decode), "
                             "5 (engine), 5small (engine, 64 x 128 tokens), 5fp8 (engine, fp8 "
                             "KV cache), step (one config-5 decode iteration, 32 x 1024 "
                             "tokens: ms, algorithmic bytes, fraction of HBM), ew (elementwise "
                             "kernels), kv (KV write), dense (dense-cache attention), linear "
                             "(decode projections and argmax), gemm (prefill projections on hipBLASLt), "
                             "ceiling (read-only HBM probe: sequential and shuffled 32 KB pages), "
                             "cases (the reference's kernel-bench shapes), copy (device copy_), "
                             "pfocc (prefill items of 16 tiles on half and on all of the CUs)")
    parser.add_argument("--no-cpu", action="store_true")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build's hot path (paged attention) is a "
              "single-GPU kernel and no multi-GPU figure is produced; run with --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    from mini_vllm.kernels import ops
    from mini_vllm.kernels.extension import load_extension
    from mini_vllm.workloads import prefill_flops

    # Every measured call must run on the kernels: a decline raises instead of timing
    # the PyTorch path.
    ops.set_strict(True)
    ext = load_extension()
    log(f"library {ext.path}; device {torch.cuda.get_device_name(0)}")

    sampler = ClockSampler().__enter__()
    log("config 2: building inputs")
    batches = rotated_batches(2, args.copies)
    b = batches[0]
    kv_bytes = b.kv_bytes()
    plan = ext.paged_attention_plan(b.q.shape[0], len(b.contexts), 16, 8, 128, 16, 1,
                                    b.max_context_len, b.q.dtype, b.key_pool.dtype)
    log(f"config 2: K+V {kv_bytes / 1e6:.1f} MB per step, plan {plan}")
    ms = run_paged(batches, args.steps, args.warmup)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    log(f"config 2: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s)")
    from mini_vllm.kernels import ops as _ops

    loaded = sampler.under_load(lambda i: _ops.paged_attention(
        *batches[i % len(batches)].args(), use_cuda=True), ms)
    log(f"config 2: clocks while it runs (amd-smi): {loaded}")

    extras = {}
    wanted = set() if args.skip_extras else {e.strip() for e in args.extras.split(",") if e.strip()}
    del batches
    torch.cuda.empty_cache()
    if "3" in wanted:
        log("config 3: building inputs")
        pf = rotated_batches(3, 2)
        flops = prefill_flops(pf[0])
        pms = run_paged(pf, max(10, args.steps // 2), 3)
        tflops = flops / (pms * 1e-3) / 1e12
        extras["config3_prefill"] = {
            "ms_per_call": round(pms, 4), "gflop": round(flops / 1e9, 3),
            "tflops": round(tflops, 2), "frac_of_bf16_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
        log(f"config 3: {pms * 1e3:.1f} us, {tflops:.1f} TFLOP/s")
        del pf
        torch.cuda.empty_cache()
    if "3fp8" in wanted:
        log("config 3 over an fp8 pool: building inputs")
        pf = rotated_batches(3, 2, kv_dtype=torch.float8_e4m3fn)
        flops = prefill_flops(pf[0])
        pms = run_paged(pf, max(10, args.steps // 2), 3)
        tflops = flops / (pms * 1e-3) / 1e12
        extras["config3_prefill_fp8kv"] = {
            "ms_per_call": round(pms, 4), "gflop": round(flops / 1e9, 3),
            "tflops": round(tflops, 2), "frac_of_bf16_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
        log(f"config 3 fp8 KV: {pms * 1e3:.1f} us, {tflops:.1f} TFLOP/s")
        del pf
        torch.cuda.empty_cache()
    if "4" in wanted:
        log("config 4: building inputs")
        f8 = rotated_batches(4, 2)
        f8_bytes = f8[0].kv_bytes() + f8[0].scale_bytes()
        fms = run_paged(f8, max(10, args.steps // 2), 3)
        fgbs = f8_bytes / (fms * 1e-3) / 1e9
        extras["config4_fp8_decode"] = {
            "ms_per_call": round(fms, 4), "bytes": f8_bytes, "gbs": round(fgbs, 1),
            "frac_of_hbm_peak": round(fgbs / HBM_PEAK_GBS, 4)}
        log(f"config 4: {fms * 1e3:.1f} us, {fgbs:.0f} GB/s")
        del f8
        torch.cuda.empty_cache()
    if "ew" in wanted:
        extras["elementwise"] = run_elementwise()
    if "kv" in wanted:
        extras["kv_write"] = run_kv_write()
    if "dense" in wanted:
        extras["dense_attention"] = run_dense()
    if "linear" in wanted:
        extras["decode_projections"] = run_linear()
    if "gemm" in wanted:
        extras["prefill_projections"] = run_prefill_gemm()
    if "5" in wanted:
        log("config 5: Qwen3-0.6B-shaped engine, 256 requests x 256 tokens")
        extras["config5_engine"] = run_engine()
        log(f"config 5 (decode graphs on): {extras['config5_engine']}")
    if "step" in wanted:
        extras["decode_step"] = run_decode_step()
        log(f"decode step (32 sequences, 1024-token prompts): {extras['decode_step']}")
        torch.cuda.empty_cache()
    if "pfocc" in wanted:
        extras["prefill_occupancy"] = run_prefill_occupancy()
        log(f"prefill occupancy: {extras['prefill_occupancy']}")
    if "5small" in wanted:
        # A shorter engine run (64 requests x 128 tokens), sized for a kernel trace.
        extras["config5_engine_small"] = run_engine(requests=64, max_tokens=128)
        log(f"config 5 small: {extras['config5_engine_small']}")
    if "5fp8" in wanted:
        extras["config5_engine_fp8kv"] = run_engine(kv_dtype=torch.float8_e4m3fn)
        log(f"config 5 with an fp8 KV cache: {extras['config5_engine_fp8kv']}")
        torch.cuda.empty_cache()
    if "copy" in wanted:
        extras["copy_ceiling_gbs"] = round(copy_ceiling(1 << 30), 1)
        log(f"copy_ ceiling {extras['copy_ceiling_gbs']} GB/s (1 GiB device-to-device copies)")
    if "ceiling" in wanted:
        ceil = read_ceiling()
        ceil["config2_frac_of_shuffled"] = round(gbs / ceil["shuffled_pages_gbs"], 4)
        ceil["config2_frac_of_sequential"] = round(gbs / ceil["sequential_gbs"], 4)
        extras["read_ceiling"] = ceil
    if "cases" in wanted:
        extras["kernel_cases"] = run_kernel_cases()
    sampler.__exit__(None, None, None)
    clocks = sampler.report()
    log(f"gpu clocks over the GPU legs: {clocks}")
    if clocks.get("throttled"):
        log("WARNING: the GPU ran below half its clocks during this run; its numbers measure "
            "the power state, not the code")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle on host cores)")
        cpu = cpu_baseline()

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, shuffled block tables)",
        "config": {
            "workload": "BASELINE config 2: paged decode, batch 64, ctx U[512,4096] seed 0, "
                        "GQA 16q/8kv, head_dim 128, 16-token pages",
            "batch": len(b.contexts),
            "total_context_tokens": sum(b.contexts),
            "kv_bytes_per_step": kv_bytes,
            "rotated_pool_copies": args.copies,
            "split_plan": plan,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
        "cpu_baseline": cpu,
        "gpu_clocks": clocks,
        "extras": extras,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
