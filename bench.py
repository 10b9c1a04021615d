"""Benchmark of the fused sampling / verification path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints one JSON line with the headline
metric: fused decode-sample microseconds per step and achieved HBM GB/s at B=64, V=128256 bf16
(config 1, ``UnshardedFusedSingular.autoregressive``), plus ``roofline`` for the dominant kernel
(the tile kernel, timed live with HIP events on the launch stream; HBM traffic per launch from the
committed FETCH_SIZE / WRITE_SIZE summary in ``profiles/``) and ``cpu_baseline`` (the CPU
restatement of the reference's PyTorch path from ``oracle/``, timed on a bounded sample of the
same workload).

The module also defines the synthetic workloads of all five configurations; the parity tests
import them. Logits follow one generator: x ~ N(0, 3^2) plus 1-16 spikes of U[10, 20] per row,
seeded with 1000 + config index, drawn on the CPU.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from dataclasses import dataclass
from pathlib import Path
from typing import List, Optional

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sonic-sampler_amd"))

import torch  # noqa: E402

BF16 = torch.bfloat16
I32 = torch.int32
I64 = torch.int64
HBM_PEAK_GBS = 8000.0


# ------------------------------------------------------------------------------------------------
# Synthetic workloads
# ------------------------------------------------------------------------------------------------

def spiked_logits(rows: int, vocab: int, seed: int, dtype=BF16) -> torch.Tensor:
    """N(0, 3^2) logits with 1-16 spikes of +U[10, 20] per row (CPU)."""

    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(rows, vocab, generator=g, dtype=torch.float32) * 3.0
    counts = torch.randint(1, 17, (rows,), generator=g)

    for r in range(rows):

        cols = torch.randperm(vocab, generator=g)[: int(counts[r])]
        x[r, cols] += torch.empty(len(cols)).uniform_(10.0, 20.0, generator=g)

    return x.to(dtype)


def c0_inputs(seed: int = 1000):
    """Config 0: UnshardedBoundedTopK, B=8, V=32000 fp32, k=32."""

    return spiked_logits(8, 32000, seed, torch.float32), 32


@dataclass
class SingularWorkload:
    logits: torch.Tensor          # [R, V] bf16 (CPU)
    buffers: object               # SamplingBuffers (CPU)
    vocab: int
    max_top_logprobs: int
    timestep: int = 0
    slot_mapping: Optional[torch.Tensor] = None
    d2t: Optional[torch.Tensor] = None
    tokens: Optional[torch.Tensor] = None
    target_vocab: Optional[int] = None


def c1_workload(seed: int = 1001, batch: int = 64, vocab: int = 128256) -> SingularWorkload:
    """Config 1: autoregressive decode with heterogeneous per-row parameters."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, ScopedIndicators

    g = torch.Generator("cpu").manual_seed(seed + 7)
    logits = spiked_logits(batch, vocab, seed)
    bf = lambda v: float(torch.tensor(v).to(BF16))  # noqa: E731

    temperature = [bf(float(torch.empty(1).uniform_(0.5, 1.5, generator=g))) for _ in range(batch)]
    top_k = [[128, 20, 50][int(torch.randint(0, 3, (1,), generator=g))] for _ in range(batch)]
    top_p = [bf(float(torch.empty(1).uniform_(0.8, 1.0, generator=g))) for _ in range(batch)]
    min_p = [[0.0, bf(0.05)][int(torch.randint(0, 2, (1,), generator=g))] for _ in range(batch)]
    biases = []

    for _ in range(batch):

        ids = torch.randperm(vocab, generator=g)[:16]
        vals = torch.empty(16).uniform_(-5.0, 5.0, generator=g)
        biases.append({int(i): bf(float(v)) for i, v in zip(ids, vals)})

    scoped = ScopedIndicators.from_params(
        size=batch, timesteps=1,
        multiplicative=[bf(1.1)] * batch, frequency=[bf(0.2)] * batch, presence=[bf(0.3)] * batch,
        biases=biases, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
        top_logprobs=[5] * batch,
    )

    buffers = SamplingBuffers.default(size=batch, timesteps=1, vocab_size=vocab, device="cpu", noise=False)
    buffers.flags = Flags.from_scoped(scoped, device="cpu")
    buffers.weights.gumbel.target.exponential_(1.0, generator=g).log_()
    buffers.temperature.copy_(torch.tensor(temperature).to(BF16))
    buffers.top_k.copy_(torch.tensor(top_k, dtype=I32))
    buffers.top_p.copy_(torch.tensor(top_p).to(BF16))
    buffers.min_p.copy_(torch.tensor(min_p).to(BF16))
    buffers.top_logprobs.fill_(5)
    rep = buffers.repetition
    rep.multiplicative.fill_(1.1)
    rep.frequency.fill_(0.2)
    rep.presence.fill_(0.3)

    history = torch.randint(0, vocab, (batch, 512), generator=g)
    rep.counts.decode.zero_().scatter_add_(1, history, torch.ones_like(history, dtype=I32))

    for r, bias in enumerate(biases):

        for i, v in bias.items():

            buffers.bias[r, i] = v

    return SingularWorkload(logits=logits, buffers=buffers, vocab=vocab, max_top_logprobs=5)


@dataclass
class MultistepWorkload:
    logits: torch.Tensor          # flat [rows, V] bf16 (CPU)
    drafted: torch.Tensor         # flat [rows] int32
    buffers: object
    cu_seqlens: List[int]
    lookahead: int
    vocab: int
    max_top_logprobs: int
    probabilities: Optional[torch.Tensor] = None   # [B, gamma, V] bf16
    varlen: bool = False


def c2_workload(seed: int = 1002, batch: int = 128, gamma: int = 4, vocab: int = 151936) -> MultistepWorkload:
    """Config 2: greedy verification, drafts = target argmax w.p. 0.7 else uniform in [1, V)."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    n = gamma + 1
    g = torch.Generator("cpu").manual_seed(seed + 7)
    logits = spiked_logits(batch * n, vocab, seed)
    argmax = logits.float().argmax(dim=-1)
    keep = torch.rand(batch * n, generator=g) < 0.7
    other = torch.randint(1, vocab, (batch * n,), generator=g)
    drafted = torch.where(keep, argmax, other).to(I32)

    buffers = SamplingBuffers.default(size=batch, timesteps=n, vocab_size=vocab, device="cpu", noise=False)
    buffers.flags = Flags.from_values(batch, n, Indicator.GREEDY, device="cpu")
    buffers.top_k.fill_(1)

    return MultistepWorkload(logits=logits, drafted=drafted, buffers=buffers,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma,
                             vocab=vocab, max_top_logprobs=5)


def c3_workload(seed: int = 1003, batch: int = 64, gamma: int = 7, vocab: int = 128256,
                lengths: Optional[List[int]] = None) -> MultistepWorkload:
    """Config 3: stochastic verification, variable lookahead U{1..7}, top-20 logprobs.

    ``lengths`` (rows per request, each within [2, gamma + 1]) fixes the request layout; by default
    it is drawn from the seed."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    g = torch.Generator("cpu").manual_seed(seed + 7)
    drawn = (torch.randint(1, gamma + 1, (batch,), generator=g) + 1).tolist()
    lengths = drawn if lengths is None else list(lengths)
    cu = [0]

    for length in lengths:

        cu.append(cu[-1] + length)

    rows = cu[-1]
    logits = spiked_logits(rows, vocab, seed)

    probabilities = torch.zeros(batch, gamma, vocab, dtype=BF16)
    drafted = torch.zeros(rows, dtype=I32)

    for b in range(batch):

        for i in range(lengths[b] - 1):

            noisy = logits[cu[b] + i].float() + torch.randn(vocab, generator=g)
            q = torch.softmax(noisy, dim=-1).to(BF16)
            probabilities[b, i] = q
            token = 0

            while token == 0:

                token = int(torch.multinomial(q.float(), 1, generator=g))

            drafted[cu[b] + i] = token

        drafted[cu[b + 1] - 1] = int(torch.randint(1, vocab, (1,), generator=g))

    indicator = Indicator.TOP_K_LOGPROBS
    buffers = SamplingBuffers.default(size=batch, timesteps=gamma + 1, vocab_size=vocab, device="cpu",
                                      noise=False)
    buffers.flags = Flags.from_values(batch, gamma + 1, indicator, device="cpu")
    buffers.top_logprobs.fill_(20)
    weights = buffers.weights
    weights.gumbel.target.exponential_(1.0, generator=g).log_()
    weights.uniform.uniform_(torch.finfo(BF16).tiny, 1.0, generator=g)

    return MultistepWorkload(logits=logits, drafted=drafted, buffers=buffers, cu_seqlens=cu,
                             lookahead=gamma, vocab=vocab, max_top_logprobs=20,
                             probabilities=probabilities, varlen=True)


def c4_workload(seed: int = 1004, rows: int = 256, slots: int = 512, gamma: int = 4,
                draft_vocab: int = 32000, target_vocab: int = 262144,
                timestep: int = 3) -> SingularWorkload:
    """Config 4: drafting with d2t (32000 -> 262144), 256 of 512 slots, 5% grammar."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    g = torch.Generator("cpu").manual_seed(seed + 7)
    logits = spiked_logits(rows, draft_vocab, seed)
    d2t = torch.randperm(target_vocab, generator=g)[:draft_vocab].to(I32)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(I32)

    buffers = SamplingBuffers.default(size=slots, timesteps=gamma + 1, vocab_size=target_vocab,
                                      device="cpu", noise=False)
    buffers.flags = Flags.from_values(slots, gamma + 1, Indicator.GRAMMAR, Indicator.GRAMMAR, device="cpu")

    words = target_vocab // 32
    bits = torch.rand(rows, target_vocab, generator=g) < 0.05
    spikes = logits.float().argmax(dim=-1)
    bits[torch.arange(rows), d2t[spikes].to(I64)] = True
    packed = (bits.view(rows, words, 32).to(I64) << torch.arange(32, dtype=I64)).sum(-1)
    grammar = buffers.grammar.view(I32)

    for r in range(rows):

        grammar[int(slot_mapping[r]), timestep] = (packed[r] - ((packed[r] >> 31) << 32)).to(I32)

    buffers.weights.gumbel.draft[:, timestep].exponential_(1.0, generator=g).log_()
    tokens = torch.randint(1, target_vocab, (rows, gamma + 1), generator=g).to(I32)

    return SingularWorkload(logits=logits, buffers=buffers, vocab=draft_vocab, max_top_logprobs=5,
                            timestep=timestep, slot_mapping=slot_mapping, d2t=d2t, tokens=tokens,
                            target_vocab=target_vocab)


def to_device(buffers, device):
    """A device copy of a CPU SamplingBuffers (same layout)."""

    import dataclasses

    from sonic_sampler.base import SliceBuffer
    from sonic_sampler.base.tensor import PrefixContiguousTensor, prefix_contiguous
    from sonic_sampler.core.flags import Flags

    def move(obj):

        if isinstance(obj, Flags):

            packed = obj.packed.T.contiguous().to(device).T if obj.packed.stride(0) == 1 else obj.packed.to(device)

            return Flags(indicators=obj.indicators, pinned=obj.pinned, packed=packed, layout=obj.layout)

        if isinstance(obj, SliceBuffer):

            kwargs = {f.name: move(getattr(obj, f.name)) for f in dataclasses.fields(obj)}

            return obj.__class__(**kwargs)

        if isinstance(obj, PrefixContiguousTensor):

            return prefix_contiguous(obj.as_subclass(torch.Tensor).to(device))

        if isinstance(obj, torch.Tensor):

            return obj if obj.device.type == "cpu" and obj.is_pinned() else obj.to(device)

        return obj

    return move(buffers)


# ------------------------------------------------------------------------------------------------
# Measurement
# ------------------------------------------------------------------------------------------------

C1_BYTES_PER_ELEMENT = 2 + 4 + 4 + 2   # logits, context counts, decode counts, bias


def c1_algorithmic_bytes(batch: int, vocab: int, top_logprobs: int = 5) -> int:
    """HBM bytes one fused autoregressive call must move at config 1."""

    streamed = batch * vocab * C1_BYTES_PER_ELEMENT
    gathers = batch * 128 * 2                           # Gumbel noise gathers (buffer mode)
    outputs = batch * (4 + 2 + top_logprobs * 6 + 4)    # token, logprob, top-Z, count update

    return streamed + gathers + outputs


def c1_tile_bytes(batch: int, vocab: int) -> int:
    """Algorithmic HBM bytes of one tile-kernel launch at config 1: every element's logit,
    context count, decode count and bias, read once."""

    return batch * vocab * C1_BYTES_PER_ELEMENT


TILE_KERNEL = "singular_tiles_kernel<16, 0>"
TRAFFIC_SUMMARY = ROOT / "profiles" / "singular_tiles_c1_traffic.txt"


def measured_traffic(kernel: str, batch: int, vocab: int) -> Optional[int]:
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE / WRITE_SIZE summary
    (counter KiB scaled by the copy-kernel calibration factor), or None when the summary is absent
    or was taken on another workload."""

    if not TRAFFIC_SUMMARY.exists():

        return None

    fields = {}

    for line in TRAFFIC_SUMMARY.read_text().splitlines():

        key, sep, value = line.partition(":")

        if sep and key.strip() and not key.startswith("#"):

            fields[key.strip()] = value.strip()

    try:

        if fields["kernel"] != kernel or int(fields["rows"]) != batch or int(fields["vocab"]) != vocab:

            return None

        return int(fields["traffic_bytes_per_launch"])

    except (KeyError, ValueError):

        return None


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo describes it: the model name plus the family / model /
    stepping numbers (which identify the part when a virtual machine shortens the name), and the
    logical CPUs this process may use."""

    fields = {}

    try:

        for line in Path("/proc/cpuinfo").read_text().splitlines():

            key, _, value = line.partition(":")
            key = key.strip()

            if key in ("model name", "cpu family", "model", "stepping", "vendor_id") and key not in fields:

                fields[key] = value.strip()

            if not line.strip() and fields:

                break

    except OSError:

        pass

    name = fields.get("model name") or platform.processor() or platform.machine()
    ids = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields)
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()

    return f"{name} ({ids}; {usable} logical CPUs usable)" if ids else f"{name} ({usable} logical CPUs usable)"


def cpu_baseline_c1(workload: SingularWorkload, budget_s: float = 15.0) -> dict:
    """The reference's PyTorch path restated in ``oracle/batch.py``, one call over the whole
    config-1 batch (as the reference's ``NaiveSampler`` runs it), timed on the host cores with the
    reference's own bounded top-128, ``logits.topk(k=128)`` (``core/naive.py:336``): one warm-up
    call, then calls until about ``budget_s`` seconds have passed (at least 3). The stable-sort
    formulation the parity tests use (ties to the lowest index) is timed the same way over a
    third of the budget and reported beside it."""

    from oracle import batch
    from oracle import sampler as oracle

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    state = oracle.State.from_buffers(workload.buffers)

    def median_us(bounded: str, budget: float):

        def run():

            batch.singular(workload.logits, state, max_top_logprobs=5, bounded=bounded)

        run()
        times = []
        t_end = time.perf_counter() + budget

        while len(times) < 3 or time.perf_counter() < t_end:

            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)

        return round(statistics.median(times) * 1e6, 1), len(times)

    value, calls = median_us("topk", budget_s)
    sorted_value, sorted_calls = median_us("sort", budget_s / 3)
    rows = workload.logits.size(0)

    return {
        "value": value,
        "unit": "us/step",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "stable_sort_value": sorted_value,
        "sample": f"oracle/batch.py singular over all {rows} rows of config 1 (one batched call with the "
                  f"reference's logits.topk(k=128), median of {calls} calls after 1 warm-up; "
                  f"stable_sort_value: the stable-sort top-128 of the parity oracle, median of "
                  f"{sorted_calls} calls); CPU: {cpu_model()}",
    }


MALL_BYTES = 256 << 20


def rotation_sets(bytes_per_set: int) -> int:
    """Input sets to rotate so that together they exceed the 256 MB MALL by a quarter: a set's
    data is then evicted before it comes round again, and steps read HBM, not the cache."""

    return max(3, -(-int(1.25 * MALL_BYTES) // max(1, bytes_per_set)))


def _queue_behind_sleep(ms: float = 60.0) -> None:
    """Keeps the GPU busy while the host enqueues the timed launches, so that they run back to
    back and each event pair brackets exactly the launches between its two records."""

    torch.cuda._sleep(int(ms * 1e-3 * 2.4e9))


def run_bench(steps: int, warmup: int, sets: Optional[int] = None, cpu_baseline: bool = True,
              philox: bool = True, block_n: Optional[int] = None) -> dict:

    from sonic_sampler import _native
    from sonic_sampler.interface import UnshardedFusedSingular

    device = torch.device("cuda:0")
    base = c1_workload()
    batch, vocab = base.logits.shape
    sets = sets or rotation_sets(c1_tile_bytes(batch, vocab))

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch,
                                                max_top_logprobs=5, block_size=block_n, device=device)
    inputs = []

    for i in range(sets):

        work = c1_workload(seed=1001 + 100 * i) if i else base
        inputs.append((work.logits.to(device), to_device(work.buffers, device)))

    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def step(i: int, tile_events=None):

        logits, buffers = inputs[i % sets]

        return sampler.autoregressive(logits, buffers, update_counts=True, logprobs=True,
                                      philox_seed=1234 if philox else None, philox_offset=i,
                                      tile_events=tile_events)

    for i in range(warmup):

        step(i)

    torch.cuda.synchronize()

    # Eager launches queued back to back: per-step time from event pairs on the launch stream.
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    _queue_behind_sleep(max(60.0, steps * 0.3))

    for i in range(steps):

        events[i][0].record(stream)
        step(i)
        events[i][1].record(stream)

    torch.cuda.synchronize()
    launch_us = [a.elapsed_time(b) * 1e3 for a, b in events]
    kernel_us = _time_back_to_back(step, steps)

    # Host cost of one eager call (argument resolution + two launches), with the GPU idle at the
    # start so that nothing but the enqueue is timed.
    enqueue = []

    for i in range(min(steps, 50)):

        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step(i)
        enqueue.append(time.perf_counter() - t0)

    torch.cuda.synchronize()

    # The tile kernel inside the full step, from events its own dispatch records at its start and
    # end (a second pass: recording them adds to each step, so the step time above runs without
    # them); reported beside the tiles-only timing below.
    tile_events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(steps)]

    for pair in tile_events:

        _native.event_pair(pair)

    torch.cuda.synchronize()
    _queue_behind_sleep(max(60.0, steps * 0.3))

    for i in range(steps):

        step(i, tile_events[i])

    torch.cuda.synchronize()
    tile_dispatch_us = statistics.mean(a.elapsed_time(b) * 1e3 for a, b in tile_events)

    # The tile kernel's average launch duration: the tile stage alone (`stage="tiles"`, the same
    # arguments and input rotation), launched back to back between one event pair behind a GPU
    # sleep. The dispatch events above put marker packets around every launch, whose cache
    # actions add about 1.3 us to each; this measure has none inside the timed region.
    def tiles_only(i: int):

        from sonic_sampler.base.tensor import plain_view
        from sonic_sampler.interface.functional.singular import fused_singular

        logits, buffers = inputs[i % sets]
        pen = buffers.repetition
        return fused_singular(
            logits=logits, indicators=buffers.flags.target, max_top_logprobs=5, update_counts=True,
            return_logprobs=True, block_n=sampler.tuning(batch)[2], scratchpad=sampler.scratchpad,
            grammar=plain_view(buffers.grammar, 0), context_counts=pen.counts.context,
            decode_counts=pen.counts.decode, repetition_penalties=pen.multiplicative,
            frequency_penalties=pen.frequency, presence_penalties=pen.presence, logit_bias=buffers.bias,
            temperature=buffers.temperature, top_k=buffers.top_k, top_p=buffers.top_p,
            min_p=buffers.min_p, top_k_logprobs=buffers.top_logprobs,
            philox_seed=1234 if philox else None, philox_offset=i,
            gumbel_noise=None if philox else plain_view(buffers.weights.gumbel.target, 0), stage="tiles")

    for i in range(warmup):

        tiles_only(i)

    tile_kernel_us = _time_back_to_back(tiles_only, steps)

    graph_us, graph_single_us, graph_median_us = _time_graphs(step, steps, sets)

    algorithmic = c1_algorithmic_bytes(batch, vocab)
    tile_bytes = c1_tile_bytes(batch, vocab)
    achieved = tile_bytes / (tile_kernel_us * 1e-6) / 1e9
    traffic = measured_traffic(TILE_KERNEL, batch, vocab)

    result = {
        "metric": "fused decode-sample us/step + achieved HBM GB/s, B=64 V=128256 bf16",
        "value": round(kernel_us, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(kernel_us * 1e-3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (spiked N(0,3^2) logits, config-1 sampling parameters, Philox noise)",
        "config": {
            "workload": "config 1: UnshardedFusedSingular.autoregressive B=64 V=128256 bf16, "
                        "penalties + bias + temperature + top-k/top-p/min-p + Gumbel-max, "
                        "logprobs + top-5, update_counts; one tile launch + one row launch per step",
            "rows": batch,
            "vocab": vocab,
            "input_sets_rotated": sets,
            "rotated_bytes": sets * c1_tile_bytes(batch, vocab),
            "algorithmic_bytes_per_step": algorithmic,
            "step_hbm_gbs": round(algorithmic / (kernel_us * 1e-6) / 1e9, 1),
            "step_hbm_frac": round(algorithmic / (kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "rows_per_s": round(batch / (kernel_us * 1e-6), 1),
            "event_pair_us_per_step": round(statistics.mean(launch_us), 3),
            "median_event_pair_us": round(statistics.median(launch_us), 3),
            "tile_kernel_us": round(tile_kernel_us, 3),
            "tile_kernel_dispatch_events_us": round(tile_dispatch_us, 3),
            "graph_replay_us_per_step": round(graph_us, 3),
            "graph_replay_single_step_us": round(graph_single_us, 3),
            "graph_replay_median_us": round(graph_median_us, 3),
            "host_us_per_eager_call": round(statistics.median(enqueue) * 1e6, 1),
        },
        "roofline": {
            "kernel": TILE_KERNEL,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": tile_bytes,
            "traffic": traffic,
        },
    }

    if cpu_baseline:

        sys.path.insert(0, str(ROOT))
        result["cpu_baseline"] = cpu_baseline_c1(base)

    return result


def _time_back_to_back(step, steps: int) -> float:
    """Microseconds per step of `steps` eager steps queued back to back: one event pair brackets
    all of them (queued behind a GPU sleep, so that the host's enqueue time is not measured). An
    event pair around every step would add its two marker packets, and the cache actions they
    force at the kernel boundaries, to every step: about 4 us at config 1."""

    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    _queue_behind_sleep(max(60.0, steps * 0.3))
    start.record(stream)

    for i in range(steps):

        step(i)

    end.record(stream)
    torch.cuda.synchronize()

    return start.elapsed_time(end) * 1e3 / steps


def _time_graphs(step, steps: int, sets: int) -> tuple:
    """Microseconds per step replayed from hipGraphs, back to back behind a GPU sleep: (a) one
    graph holding the steps of every input set in turn, replayed steps // sets times, (b) one
    graph per step, and (c) the median of (b)'s replays timed one by one. A graph launch costs about 4 us of GPU time of its own, which (b) pays on every
    step; an engine's graph holds its whole decode step (forward pass and sampling) and pays it
    once per step whatever the sampler, so (a) is the sampler's share."""

    stream = torch.cuda.current_stream()
    whole = torch.cuda.CUDAGraph()

    with torch.cuda.graph(whole):

        for i in range(sets):

            step(i)

    singles = []

    for i in range(sets):

        g = torch.cuda.CUDAGraph()

        with torch.cuda.graph(g):

            step(i)

        singles.append(g)

    def timed(replays, launch) -> float:

        for i in range(3):

            launch(i)

        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        _queue_behind_sleep(max(60.0, steps * 0.05))
        start.record(stream)

        for i in range(replays):

            launch(i)

        end.record(stream)
        torch.cuda.synchronize()

        return start.elapsed_time(end) * 1e3

    rounds = max(1, steps // sets)
    whole_us = timed(rounds, lambda i: whole.replay()) / (rounds * sets)
    single_us = timed(steps, lambda i: singles[i % sets].replay()) / steps

    # the measure of the baseline's plan: the median over at least 200 single-step replays, each
    # bracketed by its own event pair (queued back to back behind a GPU sleep)
    replays = max(200, steps)
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(replays)]
    torch.cuda.synchronize()
    _queue_behind_sleep(max(60.0, replays * 0.05))

    for i, (a, b) in enumerate(pairs):

        a.record(stream)
        singles[i % sets].replay()
        b.record(stream)

    torch.cuda.synchronize()
    median_us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in pairs)

    return whole_us, single_us, median_us


def _time_steps(step, steps: int, warmup: int, sets: int, tiles: bool = False) -> dict:
    """Eager timing (launches queued back to back; per-step event pairs as a second figure) and
    hipGraph replay timing of `step(i)`. With `tiles`, `step(i, events)` also takes an event pair
    that the tile kernel's own dispatch records, and a second pass times the tile kernel alone."""

    stream = torch.cuda.current_stream()

    for i in range(warmup):

        step(i)

    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    _queue_behind_sleep(max(60.0, steps * 0.3))

    for i in range(steps):

        events[i][0].record(stream)
        step(i)
        events[i][1].record(stream)

    torch.cuda.synchronize()
    eager = [a.elapsed_time(b) * 1e3 for a, b in events]
    back_to_back = _time_back_to_back(step, steps)
    graph_us, graph_single_us, graph_median_us = _time_graphs(step, steps, sets)
    tile_us = None

    # host cost of one eager call, the GPU idle at its start
    enqueue = []

    for i in range(min(steps, 50)):

        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step(i)
        enqueue.append(time.perf_counter() - t0)

    torch.cuda.synchronize()

    if tiles:

        from sonic_sampler import _native

        tile_events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(steps)]

        for pair in tile_events:

            _native.event_pair(pair)

        torch.cuda.synchronize()
        _queue_behind_sleep(max(60.0, steps * 0.3))

        for i in range(steps):

            step(i, tile_events[i])

        torch.cuda.synchronize()
        tile_us = statistics.mean(a.elapsed_time(b) * 1e3 for a, b in tile_events)

    return {"eager_us": back_to_back, "event_pair_us": statistics.mean(eager),
            "median_event_pair_us": statistics.median(eager), "graph_us": graph_us,
            "graph_single_us": graph_single_us, "graph_median_us": graph_median_us, "tile_us": tile_us,
            "host_us": statistics.median(enqueue) * 1e6}


CONFIG_NAMES = {
    0: "config 0: UnshardedBoundedTopK B=8 V=32000 fp32 k=32",
    2: "config 2: UnshardedFusedMultistep greedy gamma=4 B=128 V=151936 bf16, logprobs (all_greedy hint: "
       "two launches)",
    3: "config 3: UnshardedFusedMultistep stochastic varlen gamma<=7 B=64 V=128256 bf16, draft "
       "probabilities, top-20 logprobs",
    4: "config 4: UnshardedFusedSingular.drafting t=3 of gamma=4, 256 of 512 slots, d2t 32000->262144, "
       "grammar, probabilities",
}


def c4_rotation(base: SingularWorkload, sets: int, device) -> list:
    """Device inputs of `sets` config-4 steps that share the large gathered planes (noise, counts,
    bias: 128 gathers per row) but stream distinct memory: every set has its own logits, its own
    copy of the grammar plane (with the bits of its own spike tokens set) and its own slot map."""

    import dataclasses

    buffers = to_device(base.buffers, device)
    d2t = base.d2t.to(device)
    rows, words = base.logits.size(0), base.target_vocab // 32
    staged = []

    for i in range(sets):

        g = torch.Generator("cpu").manual_seed(5000 + i)
        logits = base.logits if i == 0 else spiked_logits(rows, base.vocab, seed=1004 + 100 * i)
        slots = base.slot_mapping if i == 0 else torch.randperm(buffers.layout.rows, generator=g)[:rows].to(I32)
        grammar = buffers.grammar.clone()

        if i:

            spike = base.d2t[logits.float().argmax(dim=-1)].to(I64)
            word = grammar.view(I32)[slots.to(I64).to(device), base.timestep, (spike // 32).to(device)]
            bit = torch.ones_like(spike).bitwise_left_shift(spike % 32)
            bit = (bit - ((bit >> 31) << 32)).to(I32).to(device)
            grammar.view(I32)[slots.to(I64).to(device), base.timestep, (spike // 32).to(device)] = word | bit

        probs = torch.zeros(buffers.layout.rows, base.target_vocab, dtype=BF16, device=device)
        staged.append((logits.to(device), dataclasses.replace(buffers, grammar=grammar),
                       base.tokens.to(device), probs, slots.to(device), d2t))

    return staged


def run_config(config: int, steps: int, warmup: int, sets: Optional[int] = None,
               block_n: Optional[int] = None) -> dict:
    """Timing of one of the other configurations (their parity is covered by the GPU tests).
    Input sets rotate so that together they exceed the 256 MB MALL (rotation_sets)."""

    from sonic_sampler.interface import UnshardedBoundedTopK, UnshardedFusedMultistep, UnshardedFusedSingular

    device = torch.device("cuda:0")
    per_set = {0: 8 * 32000 * 4, 2: 128 * 5 * 151936 * 2, 3: 300 * 128256 * 2,
               4: 256 * 32000 * 2 + 256 * 8192 * 4}
    sets = sets or rotation_sets(per_set[config])

    if config == 0:

        inputs = [c0_inputs(seed=1000 + 100 * i)[0].to(device) for i in range(sets)]
        topk = UnshardedBoundedTopK.initialize(vocab_size=32000, batch_size=8, k=32, block_size=block_n,
                                               device=device)
        step = lambda i: topk(inputs[i % sets])  # noqa: E731
        rows, algorithmic = 8, 8 * 32000 * 4 + 8 * 32 * 8

    elif config in (2, 3):

        makers = {2: c2_workload, 3: c3_workload}
        works = [makers[config](seed=1000 + config + 100 * i) for i in range(sets)]
        batch = len(works[0].cu_seqlens) - 1
        verifier = UnshardedFusedMultistep.initialize(vocab_size=works[0].vocab, lookahead=works[0].lookahead,
                                                      batch_size=batch, max_top_logprobs=works[0].max_top_logprobs,
                                                      block_size=block_n, device=device)
        staged = []

        for w in works:

            buffers = to_device(w.buffers, device)
            probs = w.probabilities.to(device) if w.probabilities is not None else None

            if w.varlen:

                logits, tokens = w.logits.to(device), w.drafted.to(device)
                cu = torch.tensor(w.cu_seqlens, dtype=I32, device=device)

            else:

                n = w.lookahead + 1
                logits, tokens, cu = w.logits.view(batch, n, -1).to(device), w.drafted.view(batch, n).to(device), None

            staged.append((logits, tokens, buffers, probs, cu))

        def step(i, tile_events=None):

            logits, tokens, buffers, probs, cu = staged[i % sets]

            # config 2's requests are all greedy, which an engine running greedy verification
            # knows: it says so, and the request stage takes the argmaxes itself
            return verifier(logits, tokens, buffers, probabilities=probs, logprobs=True, cu_seqlens=cu,
                            philox_seed=None, all_greedy=config == 2, tile_events=tile_events)

        rows = works[0].logits.size(0)
        algorithmic = rows * works[0].vocab * 2

    elif config == 4:

        w0 = c4_workload()
        rows = w0.logits.size(0)
        sampler = UnshardedFusedSingular.initialize(vocab_size=w0.vocab, batch_size=rows, lookahead=4,
                                                    max_top_logprobs=5, block_size=block_n, device=device)
        staged = c4_rotation(w0, sets, device)

        def step(i, tile_events=None):

            logits, buffers, tokens, probs, slots, d2t = staged[i % sets]

            return sampler.drafting(logits, buffers, timestep=w0.timestep, tokens=tokens, probabilities=probs,
                                    slot_mapping=slots, d2t_mapping=d2t, target_vocab=w0.target_vocab,
                                    in_place=True, tile_events=tile_events)

        words = w0.target_vocab // 32
        algorithmic = rows * w0.vocab * 2 + rows * words * 4 + w0.vocab * 4 + 2 * rows * 128 * 2

    else:

        raise ValueError(f"unknown config {config}")

    t = _time_steps(step, steps, warmup, sets, tiles=config != 0)
    us = t["eager_us"]

    return {
        "metric": f"config {config} us/step + achieved HBM GB/s",
        "value": round(us, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(us * 1e-3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32" if config == 0 else "bf16",
        "data": "synthetic (spiked N(0,3^2) logits, configuration generators of bench.py)",
        "config": {
            "workload": CONFIG_NAMES[config],
            "rows": rows,
            "input_sets_rotated": sets,
            "algorithmic_bytes_per_step": algorithmic,
            "achieved_hbm_gbs": round(algorithmic / (us * 1e-6) / 1e9, 1),
            "step_hbm_frac": round(algorithmic / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "rows_per_s": round(rows / (us * 1e-6), 1),
            "event_pair_us_per_step": round(t["event_pair_us"], 3),
            "median_event_pair_us": round(t["median_event_pair_us"], 3),
            "graph_replay_us_per_step": round(t["graph_us"], 3),
            "graph_replay_single_step_us": round(t["graph_single_us"], 3),
            "graph_replay_median_us": round(t["graph_median_us"], 3),
            "tile_kernel_us": None if t["tile_us"] is None else round(t["tile_us"], 3),
            "host_us_per_eager_call": round(t["host_us"], 1),
        },
    }


def copy_calibration(gib: float = 1.0, repeats: int = 5) -> None:
    """A plain elementwise device copy of known size (reads and writes `gib` GiB once each), to
    scale the FETCH_SIZE / WRITE_SIZE counters."""

    n = int(gib * (1 << 30)) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)

    for _ in range(repeats):

        torch.mul(src, 1.0, out=dst)

    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "repeats": repeats}))


def run_indexed_copy(steps: int, warmup: int) -> dict:
    """ss_indexed_copy (the noise staging behind GumbelNoise.stage_weights, reference
    ops/copy.py:21-127) at config 4's buffer shape: the drafter's noise rows of 256 stochastic
    slots of 512, [5, 262144] bf16 each, copied into the verifier's plane; 1.34 GB moved per call
    (671 MB read, 671 MB written), timed with an event pair around `steps` calls back to back. The
    reference states about 70% bandwidth utilisation for its kernel (ops/copy.py:91-92)."""

    from sonic_sampler import _native

    slots, timesteps, vocab, rows = 512, 5, 262144, 256
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(7)
    draft = torch.randn(slots, timesteps, vocab, dtype=torch.float32, device=dev).to(BF16)
    target = torch.zeros_like(draft)
    indices = torch.randperm(slots, generator=g)[:rows].to(dev)
    indicators = torch.zeros(slots, dtype=torch.uint16, device=dev)   # every slot stochastic

    for _ in range(warmup):

        _native.indexed_copy(draft, target, indices, indicators)

    torch.cuda.synchronize()

    if not torch.equal(target.index_select(0, indices), draft.index_select(0, indices)):

        raise RuntimeError("ss_indexed_copy did not copy the listed rows")

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()

    for _ in range(steps):

        _native.indexed_copy(draft, target, indices, indicators)

    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / steps
    moved = 2 * rows * timesteps * vocab * 2
    gbs = moved / us * 1e-3

    return {
        "metric": "ss_indexed_copy GB/s (read + write) at config 4's noise planes", "value": round(gbs, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "us_per_call": round(us, 2),
        "higher_is_better": True, "dtype": "bf16", "data": "synthetic N(0,1) noise rows",
        "config": {"workload": "GumbelNoise.stage_weights copy: 256 stochastic slots of 512, [5, 262144] bf16 rows",
                   "bytes_per_call": moved, "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                   "reference_claim": "about 70% bandwidth utilisation (ops/copy.py:91-92)"},
    }


def run_sparse_grammar(admitted: list, steps: int, warmup: int) -> dict:
    """Config 1's shape (B=64, V=128256 bf16) with a grammar mask as the rows' only processor,
    admitting `n` random tokens per row for each n of `admitted` (0: every token): below 128
    admitted tokens in a 4096-column tile, its top-128 ends in -inf ties, the case constrained
    decoding meets. Per n: the tile kernel (its own dispatch events, mean of `steps`) and the
    step (event pair around `steps` eager steps back to back). One input set, not rotated (17 MB
    of logits and grammar words fit the MALL): the figures compare admitted counts with each other
    and with the unconstrained row, not with the HBM roofline."""

    from sonic_sampler import _native
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator
    from sonic_sampler.interface import UnshardedFusedSingular

    rows, vocab = 64, 128256
    dev = torch.device("cuda:0")
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, device=dev)
    results = {}

    for n in admitted:

        g = torch.Generator("cpu").manual_seed(5)
        logits = spiked_logits(rows, vocab, 5).to(dev)
        host = SamplingBuffers.default(size=rows, timesteps=1, vocab_size=vocab, device="cpu", noise=False)
        host.flags = Flags.from_values(rows, 1, Indicator.GRAMMAR, Indicator.GRAMMAR, device="cpu")
        host.weights.gumbel.target.exponential_(1.0, generator=g).log_()
        words = (vocab + 31) // 32
        bits = torch.zeros(rows, words * 32, dtype=torch.bool)

        for r in range(rows):

            bits[r, torch.randperm(vocab, generator=g)[: n or vocab]] = True

        packed = (bits.view(rows, words, 32).to(torch.int64) << torch.arange(32, dtype=torch.int64)).sum(-1)
        host.grammar.view(torch.int32)[:, 0] = (packed - ((packed >> 31) << 32)).to(torch.int32)
        buffers = to_device(host, dev)
        step = lambda events=None: sampler.autoregressive(logits, buffers, tile_events=events)  # noqa: E731

        for _ in range(warmup):

            step()

        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]

        for pair in pairs:

            _native.event_pair(pair)

        torch.cuda.synchronize()

        for pair in pairs:

            step(pair)

        torch.cuda.synchronize()
        tile_us = statistics.mean(a.elapsed_time(b) * 1e3 for a, b in pairs)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()

        for _ in range(steps):

            step()

        end.record()
        torch.cuda.synchronize()
        results[str(n or vocab)] = {"tile_kernel_us": round(tile_us, 3),
                                    "us_per_step": round(start.elapsed_time(end) * 1e3 / steps, 3)}

    return {
        "metric": "config-1-shaped decode step with a sparse grammar: tile kernel and step us", "value": None,
        "unit": "us", "n_gpus": 1, "steps": steps, "warmup": warmup, "higher_is_better": False, "dtype": "bf16",
        "data": "synthetic (spiked N(0,3^2) logits, random admitted tokens per row)",
        "config": {"workload": "UnshardedFusedSingular.autoregressive B=64 V=128256 bf16, grammar only",
                   "admitted_tokens_per_row": results},
    }


def main(argv=None) -> int:

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="skip the CPU baseline of config 1")
    parser.add_argument("--sets", type=int, default=None,
                        help="input sets to rotate (default: enough to exceed the 256 MB MALL)")
    parser.add_argument("--buffer-noise", action="store_true",
                        help="read Gumbel noise from the buffers instead of the Philox stream")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run a 1 GiB device copy (PMC counter calibration)")
    parser.add_argument("--sparse-grammar", type=str, default=None, metavar="N,N,...",
                        help="time config 1's shape under grammars admitting N tokens per row (0: all)")
    parser.add_argument("--indexed-copy", action="store_true",
                        help="time the noise-staging copy (ss_indexed_copy) instead of a sampling config")
    parser.add_argument("--config", type=int, default=1, choices=[0, 1, 2, 3, 4],
                        help="configuration to time (1, the headline, by default)")
    parser.add_argument("--block-n", type=int, default=None,
                        help="tile width instead of the dispatch table's (tuning sweeps)")
    args = parser.parse_args(argv)

    if args.copy_calibration:

        copy_calibration()

        return 0

    if args.gpus != 1:

        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the sampling path "
              "shards by batch with no exchange, so N GPUs run N independent copies)", file=sys.stderr)

        return 2

    if args.sparse_grammar:

        admitted = [int(n) for n in args.sparse_grammar.split(",")]
        print(json.dumps(run_sparse_grammar(admitted, args.steps, args.warmup)), flush=True)

        return 0

    if args.indexed_copy:

        print(json.dumps(run_indexed_copy(args.steps, args.warmup)), flush=True)

        return 0

    if args.config != 1:

        print(json.dumps(run_config(args.config, args.steps, args.warmup, sets=args.sets, block_n=args.block_n)),
              flush=True)

        return 0

    result = run_bench(args.steps, args.warmup, sets=args.sets, cpu_baseline=not args.no_cpu_baseline,
                       philox=not args.buffer_noise, block_n=args.block_n)
    print(json.dumps(result), flush=True)

    return 0


if __name__ == "__main__":

    sys.exit(main())
