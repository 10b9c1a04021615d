"""ss_fused_singular_noalloc (static device scratch) against ss_fused_singular (caller scratchpad).

Both entry points are called through the C-ABI on identical inputs; every output must be
bit-identical. The no-allocation calls run twice in a row, the second on a smaller input (fewer
rows and tiles), so a stale candidate list left in the shared static array by the first call would
show. A call larger than the static array must be refused with SS_ERR_SCRATCH_LIMIT. After an eager
call on the device, the entry point is captured in a hipGraph and replayed over new inputs; a fresh
process whose first call on the device comes under capture must see that call refused.
"""

import ctypes
import subprocess
import sys

from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def build_case(rows, vocab, seed):

    from bench import spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers

    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=5)
    return host, spiked_logits(rows, vocab, seed=900 + seed)


def call(buffers, logits, block, static_scratch):
    """One autoregressive call with logprobs, top-5 and count updates (no synchronization)."""

    from sonic_sampler.interface.functional import fused_singular

    rep = buffers.repetition

    return fused_singular(
        logits=logits.to(DEV), indicators=buffers.flags.target, max_top_logprobs=5, update_counts=True,
        return_logprobs=True, block_n=block, grammar=buffers.grammar[:, 0],
        context_counts=rep.counts.context, decode_counts=rep.counts.decode,
        repetition_penalties=rep.multiplicative, frequency_penalties=rep.frequency,
        presence_penalties=rep.presence, logit_bias=buffers.bias, temperature=buffers.temperature,
        top_k=buffers.top_k, top_p=buffers.top_p, min_p=buffers.min_p,
        top_k_logprobs=buffers.top_logprobs, gumbel_noise=buffers.weights.gumbel.target[:, 0],
        static_scratch=static_scratch,
    )


def outputs(selection, host, rows, decode):
    """The outputs a call defines: tokens, logprobs, the written top logprobs, decode counts."""

    lp = selection.logprobs
    # top logprobs are written up to the row's limit only (per-row count, bit 0x400, non-greedy)
    written = torch.zeros(lp.top_k.tokens.shape, dtype=torch.bool)

    for r, ind in enumerate(host.flags.indicators.target[:rows]):

        if int(ind) & 0x400 and not int(ind) & 0x40:

            written[r, :min(int(host.top_logprobs[r]), 5)] = True

    return [selection.tokens.cpu(), lp.selected.cpu(), lp.top_k.tokens.cpu()[written],
            lp.top_k.logprobs.cpu()[written], decode.cpu()]


def run(host, logits, block, static_scratch):
    """One call on fresh device buffers, synchronized, and its outputs."""

    from bench import to_device

    buffers = to_device(host, DEV)
    selection = call(buffers, logits.to(DEV), block, static_scratch)
    torch.cuda.synchronize()

    return outputs(selection, host, logits.size(0), buffers.repetition.counts.decode)


def test_noalloc_matches_scratchpad_entry_point_on_consecutive_calls():

    # the second call is smaller: fewer rows and fewer tiles per row
    cases = [(48, 65536, 4096, 11), (12, 20480, 2048, 12)]
    expected = []

    for rows, vocab, block, seed in cases:

        host, logits = build_case(rows, vocab, seed)
        print(f"scratchpad entry point: rows={rows} V={vocab} block={block}", flush=True)
        expected.append(run(host, logits, block, static_scratch=False))

    for (rows, vocab, block, seed), want in zip(cases, expected):

        host, logits = build_case(rows, vocab, seed)
        print(f"static-scratch entry point: rows={rows} V={vocab} block={block}", flush=True)
        got = run(host, logits, block, static_scratch=True)

        for name, a, b in zip(("tokens", "logprobs", "top tokens", "top logprobs", "decode counts"), got, want):

            assert torch.equal(a, b), f"{name} differ at rows={rows} V={vocab}"


def test_noalloc_sharded_stages_match_the_scratchpad():
    """A tensor-parallel caller that cannot allocate: the W shards' tile stages into the static
    array (each into its slice), then the row stage over the W slices. Tokens, counts and logprobs
    equal the same stages through a caller scratchpad, bit for bit."""

    from bench import to_device
    from sonic_sampler.interface.functional import fused_singular
    from test_gpu_sharded import buffer_kwargs, outputs as shard_outputs, run_sharded

    rows, vocab, world, block = 8, 4 * 8192, 4, 2048
    host, logits = build_case(rows, vocab, seed=41)
    logits = logits.to(DEV)
    common = dict(max_top_logprobs=5, return_logprobs=True, update_counts=True)
    print(f"noalloc sharded: rows={rows} V={vocab} W={world} block={block}", flush=True)

    ref_buffers = to_device(host, DEV)
    reference = run_sharded(logits, ref_buffers, world, block, vocab, **buffer_kwargs(ref_buffers, "target", 0),
                            **common)

    buffers = to_device(host, DEV)
    kw = dict(buffer_kwargs(buffers, "target", 0), **common)
    shard = vocab // world

    for rank in range(world):

        fused_singular(logits[:, rank * shard:(rank + 1) * shard], world_size=world, local_rank=rank,
                       shard_size=shard, target_vocab=vocab, block_n=block, static_scratch=True,
                       stage="tiles", **kw)

    selection = fused_singular(logits[:, :shard], world_size=world, local_rank=0, shard_size=shard,
                               target_vocab=vocab, block_n=block, static_scratch=True, stage="rows", **kw)
    torch.cuda.synchronize()

    for want, got in zip(shard_outputs(reference, ref_buffers), shard_outputs(selection, buffers)):

        assert torch.equal(want, got)


def test_noalloc_refuses_calls_beyond_the_static_scratch():

    from sonic_sampler import _native

    lib = _native.load()
    tiles = 32
    rows = _native.STATIC_SCRATCH_BYTES // (tiles * 128 * 4) + 1
    args = _native.SingularArgs(rows=rows, vocab_size=tiles * 4096, block_n=4096)
    print(f"oversize static-scratch call: rows={rows} tiles={tiles} (checked before any launch)", flush=True)
    assert lib.ss_fused_singular_noalloc(ctypes.byref(args)) == _native.SS_ERR_SCRATCH_LIMIT
    assert b"static scratch" in lib.ss_status_string(_native.SS_ERR_SCRATCH_LIMIT)


def test_noalloc_captured_in_a_graph():
    """The device's first call is eager (a first call while its stream captures is refused); then
    the entry point is captured in a hipGraph and replayed over three input sets copied into the
    captured tensors, with eager work and synchronization between replays. Every replay must equal
    an eager ss_fused_singular call on the same inputs."""

    from bench import to_device
    from helpers import load_into

    rows, vocab, block = 16, 32768, 4096
    cases = [build_case(rows, vocab, seed) for seed in (21, 22, 23)]
    want = []

    for k, (host, logits) in enumerate(cases):

        print(f"scratchpad entry point, input set {k}: rows={rows} V={vocab}", flush=True)
        want.append(run(host, logits, block, static_scratch=False))

    buffers = to_device(cases[0][0], DEV)
    logits = cases[0][1].to(DEV)
    print("eager static-scratch call before capture", flush=True)
    call(buffers, logits, block, static_scratch=True)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    with torch.cuda.stream(side):

        call(buffers, logits, block, static_scratch=True)

    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("capturing the static-scratch call", flush=True)

    with torch.cuda.graph(graph):

        captured = call(buffers, logits, block, static_scratch=True)

    for rnd, k in enumerate([0, 2, 1, 2]):

        host, fresh = cases[k]
        load_into(buffers, host)
        logits.copy_(fresh)
        torch.cuda.synchronize()
        print(f"replay {rnd}: input set {k}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        got = outputs(captured, host, rows, buffers.repetition.counts.decode)

        for name, a, b in zip(("tokens", "logprobs", "top tokens", "top logprobs", "decode counts"), got, want[k]):

            assert torch.equal(a, b), f"{name} differ on replay {rnd} (input set {k})"


# Run in a fresh process, so that no earlier call has looked up the device's copy of the array.
FIRST_CALL_UNDER_CAPTURE = """
import sys
sys.path[:0] = %r
import torch
from bench import to_device
from test_zz_no_alloc import build_case, call, outputs, DEV
host, logits = build_case(8, 16384, 31)
buffers = to_device(host, DEV)
logits = logits.to(DEV)
call(buffers, logits, 4096, static_scratch=False)
torch.cuda.synchronize()
print("scratchpad warm-up done", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    try:
        call(buffers, logits, 4096, static_scratch=True)
        print("first call captured", flush=True)
    except RuntimeError as e:
        print("first call refused:", e, flush=True)
torch.cuda.synchronize()
want = outputs(call(to_device(host, DEV), logits, 4096, static_scratch=False), host, 8,
               torch.zeros(1))[:4]
eager = to_device(host, DEV)
got = outputs(call(eager, logits, 4096, static_scratch=True), host, 8, torch.zeros(1))[:4]
torch.cuda.synchronize()
print("eager call after refusal equal:", all(torch.equal(a, b) for a, b in zip(got, want)), flush=True)
"""


def test_noalloc_first_call_under_capture_is_refused():
    """A device's first no-allocation call must be eager: made while the stream captures, it is
    refused (status unsupported) before anything is recorded, and the next eager call works."""

    root = Path(__file__).resolve().parent.parent
    paths = [str(root), str(root / "sonic-sampler_amd"), str(root / "tests")]
    print("fresh process: first static-scratch call under capture", flush=True)
    out = subprocess.run([sys.executable, "-u", "-c", FIRST_CALL_UNDER_CAPTURE % paths],
                         capture_output=True, text=True, timeout=100)
    text = out.stdout + out.stderr

    assert out.returncode == 0, text
    assert "first call refused:" in out.stdout and "unsupported" in out.stdout.lower(), text
    assert "eager call after refusal equal: True" in out.stdout, text
