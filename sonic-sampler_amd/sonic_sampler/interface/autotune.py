"""Measures the dispatch tables for this GPU. For every (vocabulary, batch) bucket, each call kind
(``KINDS``) is timed at each compiled tile width:

- ``singular``: the fused single step with every processor on and logprobs;
- ``drafting``: the drafting step through d2t into an 8x wider target vocabulary under a grammar
  mask, timed in the buckets of draft vocabularies (at most ``DRAFT_VOCAB_MAX`` columns);
- ``multistep``: the verification at lookahead 3 with a typical verification state (temperature,
  top-k, top-p, top logprobs; ``VERIFY_INDICATOR``);
- ``topk``: the bounded top-128.

Each kind gets a table of its own (``--out`` names the shared one, which the ``singular`` kind
scores; the others are written beside it as ``<stem>_<kind>.toml``): the kinds' best widths differ
(the verification, bound by per-element instructions at two bytes per element, prefers wider tiles
than the decode step, which reads four planes per element), so one table scored over all of them
would slow each. Within a table a width's score is its worst slowdown over the kinds it serves
(time / that kind's fastest time), and the bucket gets the widest width whose score is within
``TOLERANCE`` of the best (run-to-run noise is about that size, and a wider tile means a smaller
scratchpad). ``--from-log`` scores the times of an earlier run's log again instead of measuring.

The tables have the schema of the reference's generated tables (``resources/dispatch/
sm100_k128.toml``, read by ``interface/dispatch.py``), whose priorities rank one configuration per
selection strategy; the gfx950 kernels have a single exact selection, so each bucket holds one
configuration (priority 0) and the measured times go to the log. ``TwoStageTiling`` sizes its
scratchpad for the smallest width of the vocabulary bucket (over the kinds that share it) and
launches each call at the width of the bucket of its row count.

    python -m sonic_sampler.interface.autotune --out gfx950_k128.toml [--vocab 8192,32768 --batch 1,64]
    [--kinds singular,multistep] [--from-log autotune.log]

Tile strategies and warp counts are recorded with fixed values: the gfx950 kernels have one exact
selection and 256-thread workgroups, so the tile width is the only tuned parameter.
"""

from __future__ import annotations

import argparse
import datetime
import functools
import statistics
import sys

from typing import Callable, Dict, Iterable, List, Optional

import torch

from sonic_sampler.interface.dispatch import (
    BatchBucket,
    DispatchMetadata,
    DispatchSummary,
    PriorityBucket,
    RuntimeConfig,
    VocabBucket,
    resolve_arch,
)
from sonic_sampler.ops.base import MAX_K

VOCAB_BUCKETS = (8192, 32768, 131072, 262144)
BATCH_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)
WIDTHS = (1024, 2048, 4096, 8192, 16384)
TOLERANCE = 0.02

KINDS = ("singular", "drafting", "multistep", "topk")
SHARED = "singular"  # the kind the shared table serves
LOOKAHEAD = 3
DRAFT_VOCAB_MAX = 32768
VERIFY_INDICATOR = 0x5A0  # temperature, top-k, top-p, top logprobs

Measure = Callable[[str, int, int, int], float]


@functools.lru_cache(maxsize=1)
def _workload(vocab: int, rows: int, device: str, seed: int):
    """Logits, drafted tokens and buffers of one bucket (the last one is kept, so the widths and
    kinds of a bucket share them): N(0, 3^2) logits, every processor but the grammar on."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    gen = torch.Generator(device).manual_seed(seed)
    logits = (torch.randn(rows, vocab, generator=gen, device=device) * 3).to(torch.bfloat16)
    drafted = torch.randint(1, vocab, (rows,), generator=gen, device=device, dtype=torch.int32)
    buffers = SamplingBuffers.random(size=rows, timesteps=LOOKAHEAD + 1, vocab_size=vocab, device=device,
                                     seed=seed, indicators=Indicator(0x7BE), max_top_logprobs=5)

    return logits, drafted, buffers


def _time(call: Callable[[], object], steps: int, warmup: int) -> float:
    """Median microseconds of one `call()`: the timed calls are queued behind a GPU sleep, so they
    run back to back and each event pair brackets the GPU's work on one call, not the host's time
    to issue it."""

    for _ in range(warmup):

        call()

    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(max(30.0, 0.2 * steps) * 1e-3 * 2.4e9))  # ~30 ms at 2.4 GHz

    for start, end in events:

        start.record(stream)
        call()
        end.record(stream)

    torch.cuda.synchronize()

    return statistics.median(a.elapsed_time(b) * 1e3 for a, b in events)


def measure_kind(kind: str, vocab: int, batch: int, block_n: int, *, device="cuda", steps: int = 30,
                 warmup: int = 3, seed: int = 0) -> Optional[float]:
    """Median microseconds of one call of `kind` over `batch` rows at (vocab, block_n), or None
    where the kind has no call of that size (a verification needs two rows per request; drafting
    is timed for draft vocabularies, at most DRAFT_VOCAB_MAX columns)."""

    from sonic_sampler.interface import UnshardedBoundedTopK, UnshardedFusedMultistep, UnshardedFusedSingular
    from sonic_sampler.interface.functional import fused_singular

    logits, drafted, buffers = _workload(vocab, max(batch, 2), str(device), seed)

    if kind == "singular":

        rep = buffers.repetition
        kw = dict(
            indicators=buffers.flags.target, max_top_logprobs=5, return_logprobs=True, block_n=block_n,
            grammar=buffers.grammar[:, 0], context_counts=rep.counts.context, decode_counts=rep.counts.decode,
            repetition_penalties=rep.multiplicative, frequency_penalties=rep.frequency,
            presence_penalties=rep.presence, logit_bias=buffers.bias, temperature=buffers.temperature,
            top_k=buffers.top_k, top_p=buffers.top_p, min_p=buffers.min_p, top_k_logprobs=buffers.top_logprobs,
            philox_seed=1, kernel_layout="tiles",
        )
        return _time(lambda: fused_singular(logits[:batch], **kw), steps, warmup)

    if kind == "multistep":

        if batch < 2:

            return None

        from sonic_sampler.core.flags import Flags, Indicator

        n = min(LOOKAHEAD + 1, batch)
        requests = batch // n
        rows = requests * n
        verifier = UnshardedFusedMultistep.initialize(vocab_size=vocab, lookahead=n - 1, batch_size=requests,
                                                      block_size=block_n, max_top_logprobs=5, device=device)
        view = logits[:rows].view(requests, n, vocab)
        tokens = drafted[:rows].view(requests, n)
        flags = buffers.flags
        buffers.flags = Flags.from_values(flags.layout.rows, LOOKAHEAD + 1, Indicator(VERIFY_INDICATOR),
                                          Indicator(VERIFY_INDICATOR), device=device)
        try:

            return _time(lambda: verifier(view, tokens, buffers, logprobs=True, philox_seed=1), steps, warmup)

        finally:

            buffers.flags = flags

    if kind == "topk":

        topk = UnshardedBoundedTopK.initialize(vocab_size=vocab, block_size=block_n, batch_size=batch,
                                               device=device)
        return _time(lambda: topk(logits[:batch]), steps, warmup)

    if kind == "drafting":

        if vocab > DRAFT_VOCAB_MAX:

            return None

        target, d2t, grammar = _drafting(vocab, batch, str(device), seed)
        sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch, lookahead=LOOKAHEAD,
                                                    block_size=block_n, max_top_logprobs=5, device=device)
        return _time(lambda: sampler.drafting(logits[:batch], grammar, timestep=1, tokens=None, d2t_mapping=d2t,
                                              target_vocab=target, philox_seed=1), steps, warmup)

    raise ValueError(f"unknown call kind {kind!r}")


@functools.lru_cache(maxsize=1)
def _drafting(vocab: int, rows: int, device: str, seed: int):
    """d2t into a target vocabulary 8x wider (at most 262144) and buffers whose rows allow about
    6% of it (each bit the AND of four random bits) through their grammar mask, the only processor
    on."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    target = min(8 * vocab, 262144)
    gen = torch.Generator(device).manual_seed(seed + 1)
    d2t = torch.randperm(target, generator=gen, device=device)[:vocab].to(torch.int32)
    buffers = SamplingBuffers.default(size=rows, timesteps=LOOKAHEAD + 1, vocab_size=target, device=device,
                                      noise=False)
    buffers.flags = Flags.from_values(rows, LOOKAHEAD + 1, Indicator.GRAMMAR, Indicator.GRAMMAR, device=device)
    grammar = buffers.grammar.view(torch.int32)
    draw = lambda: torch.randint(-2 ** 31, 2 ** 31, grammar.shape, generator=gen, device=device,  # noqa: E731
                                 dtype=torch.int32)
    grammar.copy_(draw() & draw() & draw() & draw())

    return target, d2t, buffers


def autotune(vocab_sizes: Iterable[int] = VOCAB_BUCKETS, batch_sizes: Iterable[int] = BATCH_BUCKETS,
             widths: Iterable[int] = WIDTHS, measure: Optional[Measure] = None, kinds: Iterable[str] = KINDS,
             k: int = MAX_K, arch: Optional[str] = None, log=None) -> DispatchSummary:
    """The dispatch table measured by `measure(kind, vocab, batch, block_n) -> microseconds or
    None` (by default `measure_kind` on the current GPU). Widths that leave fewer than two tiles
    are skipped, and so are buckets where no kind has a call (lookups there take the nearest
    bucket, or the shared table)."""

    measure = measure or measure_kind
    arch = arch or resolve_arch(None)
    vocab = PriorityBucket()

    for v in sorted(vocab_sizes):

        batches = PriorityBucket()

        for b in sorted(batch_sizes):

            usable = [w for w in widths if -(-v // w) >= 2]
            score = {w: 1.0 for w in usable}
            lines = []

            for kind in kinds:

                times = {w: measure(kind, v, b, w) for w in usable}

                if any(t is None for t in times.values()):

                    continue

                best = min(times.values())

                for w in usable:

                    score[w] = max(score[w], times[w] / best)

                lines.append(f"{kind} " + " ".join(f"{w}:{times[w]:.2f}" for w in usable))

            if not lines:

                continue

            low = min(score.values())
            pick = max(w for w in usable if score[w] <= low * (1 + TOLERANCE))

            if log is not None:

                log(f"vocab {v} batch {b}: {pick} | " + " | ".join(lines))

            config = RuntimeConfig(priority=0, block_n=pick, strategy="radix", first_warps=4, second_warps=4)
            batches.append(BatchBucket(size=b, config=[config]))

        if batches:

            vocab.append(VocabBucket(size=v, batch=batches))

    stamp = datetime.datetime.now(datetime.timezone.utc).isoformat()

    return DispatchSummary(metadata=DispatchMetadata(version=1, timestamp=f"{stamp} ({arch}, measured)"),
                           k=k, vocab=vocab)


def table_path(out: str, kind: str) -> str:
    """Where the table of `kind` goes when the shared table goes to `out`."""

    if kind == SHARED:

        return out

    stem, dot, ext = out.rpartition(".")

    return f"{stem}_{kind}.{ext}" if dot else f"{out}_{kind}"


def parse_log(lines: Iterable[str]) -> Dict[tuple, float]:
    """Times of a run's log: {(kind, vocab, batch, block_n): microseconds}, from lines
    ``vocab V batch B: pick | kind w:t w:t ... | kind ...``."""

    times = {}

    for line in lines:

        if not line.startswith("vocab ") or "|" not in line:

            continue

        head, *parts = line.strip().split(" | ")
        words = head.split()
        vocab, batch = int(words[1]), int(words[3].rstrip(":"))

        for part in parts:

            kind, *entries = part.split()

            for entry in entries:

                width, time = entry.split(":")
                times[(kind, vocab, batch, int(width))] = float(time)

    return times


def main(argv=None) -> int:

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--out", required=True, help="path of the shared TOML table to write")
    parser.add_argument("--vocab", default=",".join(map(str, VOCAB_BUCKETS)))
    parser.add_argument("--batch", default=",".join(map(str, BATCH_BUCKETS)))
    parser.add_argument("--widths", default=",".join(map(str, WIDTHS)))
    parser.add_argument("--kinds", default=",".join(KINDS))
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--from-log", default=None, help="score the times of an earlier run's log")
    args = parser.parse_args(argv)

    ints = lambda text: [int(x) for x in text.split(",") if x]  # noqa: E731
    kinds = [x for x in args.kinds.split(",") if x]

    if args.from_log:

        with open(args.from_log) as f:

            logged = parse_log(f)

        measure = lambda *key: logged.get(key)  # noqa: E731

    else:

        measure = functools.lru_cache(maxsize=None)(
            lambda *key: measure_kind(*key, steps=args.steps, warmup=args.warmup))

    for kind in kinds:

        summary = autotune(ints(args.vocab), ints(args.batch), ints(args.widths), measure=measure, kinds=[kind],
                           log=lambda line: print(line, flush=True))
        path = table_path(args.out, kind)
        summary.save(path)
        print(f"wrote {path}", flush=True)

    return 0


if __name__ == "__main__":

    sys.exit(main())
