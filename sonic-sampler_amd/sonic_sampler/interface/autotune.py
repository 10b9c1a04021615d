"""Measures a dispatch table for this GPU: for every (vocabulary, batch) bucket, the fused
single-step call (every processor on, logprobs) is timed at each compiled tile width and the widths
are written fastest first, as the priorities of the bucket's configurations. The table has the
schema of the reference's generated tables (``resources/dispatch/sm100_k128.toml``, read by
``interface/dispatch.py``); ``UnshardedFusedSingular`` / ``UnshardedFusedMultistep.initialize``
pick the priority-0 width of the bucket of their row count.

    python -m sonic_sampler.interface.autotune --out gfx950_k128.toml [--vocab 8192,32768 --batch 1,64]

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
WIDTHS = (1024, 2048, 4096, 8192)

Measure = Callable[[int, int, int], float]


@functools.lru_cache(maxsize=1)
def _workload(vocab: int, batch: int, device: str, seed: int):
    """Logits and buffers of one bucket (the last one is kept, so the widths of a bucket share
    them): N(0, 3^2) logits, every processor but the grammar on, logprobs."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    gen = torch.Generator(device).manual_seed(seed)
    logits = (torch.randn(batch, vocab, generator=gen, device=device) * 3).to(torch.bfloat16)
    buffers = SamplingBuffers.random(size=batch, timesteps=1, vocab_size=vocab, device=device, seed=seed,
                                     indicators=Indicator(0x7BE), max_top_logprobs=5)

    return logits, buffers


def measure_fused(vocab: int, batch: int, block_n: int, *, device="cuda", steps: int = 50,
                  warmup: int = 5, seed: int = 0) -> float:
    """Median microseconds of one fused autoregressive call at (vocab, batch, block_n): the timed
    calls are queued behind a GPU sleep, so they run back to back and each event pair brackets the
    GPU's work on one call, not the host's time to issue it."""

    from sonic_sampler.interface.functional import fused_singular

    logits, buffers = _workload(vocab, batch, str(device), seed)
    rep = buffers.repetition
    kw = dict(
        indicators=buffers.flags.target, max_top_logprobs=5, return_logprobs=True, block_n=block_n,
        grammar=buffers.grammar[:, 0], context_counts=rep.counts.context, decode_counts=rep.counts.decode,
        repetition_penalties=rep.multiplicative, frequency_penalties=rep.frequency,
        presence_penalties=rep.presence, logit_bias=buffers.bias, temperature=buffers.temperature,
        top_k=buffers.top_k, top_p=buffers.top_p, min_p=buffers.min_p, top_k_logprobs=buffers.top_logprobs,
        philox_seed=1, kernel_layout="tiles",
    )

    for _ in range(warmup):

        fused_singular(logits, **kw)

    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(max(30.0, 0.2 * steps) * 1e-3 * 2.4e9))  # ~30 ms at 2.4 GHz

    for start, end in events:

        start.record(stream)
        fused_singular(logits, **kw)
        end.record(stream)

    torch.cuda.synchronize()

    return statistics.median(a.elapsed_time(b) * 1e3 for a, b in events)


def autotune(vocab_sizes: Iterable[int] = VOCAB_BUCKETS, batch_sizes: Iterable[int] = BATCH_BUCKETS,
             widths: Iterable[int] = WIDTHS, measure: Optional[Measure] = None, k: int = MAX_K,
             arch: Optional[str] = None, log=None) -> DispatchSummary:
    """The dispatch table measured by `measure(vocab, batch, block_n) -> microseconds` (by default
    `measure_fused` on the current GPU). Widths that leave fewer than two tiles are skipped."""

    measure = measure or measure_fused
    arch = arch or resolve_arch(None)
    vocab = PriorityBucket()

    for v in sorted(vocab_sizes):

        batches = PriorityBucket()

        for b in sorted(batch_sizes):

            times: Dict[int, float] = {w: measure(v, b, w) for w in widths if -(-v // w) >= 2}
            ranked: List[int] = sorted(times, key=lambda w: (times[w], w))

            if log is not None:

                log(f"vocab {v} batch {b}: " + ", ".join(f"{w}: {times[w]:.2f} us" for w in ranked))

            configs = [RuntimeConfig(priority=i, block_n=w, strategy="radix", first_warps=4, second_warps=4)
                       for i, w in enumerate(ranked)]
            batches.append(BatchBucket(size=b, config=configs))

        vocab.append(VocabBucket(size=v, batch=batches))

    stamp = datetime.datetime.now(datetime.timezone.utc).isoformat()

    return DispatchSummary(metadata=DispatchMetadata(version=1, timestamp=f"{stamp} ({arch}, measured)"),
                           k=k, vocab=vocab)


def main(argv=None) -> int:

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--out", required=True, help="path of the TOML table to write")
    parser.add_argument("--vocab", default=",".join(map(str, VOCAB_BUCKETS)))
    parser.add_argument("--batch", default=",".join(map(str, BATCH_BUCKETS)))
    parser.add_argument("--widths", default=",".join(map(str, WIDTHS)))
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    args = parser.parse_args(argv)

    ints = lambda text: [int(x) for x in text.split(",") if x]  # noqa: E731
    summary = autotune(ints(args.vocab), ints(args.batch), ints(args.widths),
                       measure=lambda v, b, w: measure_fused(v, b, w, steps=args.steps, warmup=args.warmup),
                       log=lambda line: print(line, flush=True))
    summary.save(args.out)
    print(f"wrote {args.out}", flush=True)

    return 0


if __name__ == "__main__":

    sys.exit(main())
