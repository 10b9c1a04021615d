"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch

import dataclasses

from types import SimpleNamespace

from oracle import sampler as oracle
from oracle.sampler import LOGPROB_FLOOR, bf16_within


def check_singular(selection, expected, *, logprobs: bool, probabilities=None, slot_mapping=None,
                   max_knife_fraction: float = 0.05):

    tokens = selection.tokens[:, 0].cpu()
    mismatched = [r for r, e in enumerate(expected) if int(tokens[r]) != e.token]
    unexplained = [r for r in mismatched if not expected[r].knife]

    assert not unexplained, (
        f"token mismatch on non-knife-edge rows {unexplained[:8]}: "
        f"got {[int(tokens[r]) for r in unexplained[:8]]}, "
        f"expected {[expected[r].token for r in unexplained[:8]]}"
    )

    assert len(mismatched) <= max(1, int(max_knife_fraction * len(expected)))

    lp = selection.logprobs.selected.float().cpu() if logprobs and selection.logprobs else None
    top = selection.logprobs.top_k if logprobs and selection.logprobs else None
    top_tokens = top.tokens.cpu() if top is not None else None
    top_values = top.logprobs.float().cpu() if top is not None else None
    probs = probabilities.float().cpu() if probabilities is not None else None
    checked = 0

    for r, e in enumerate(expected):

        if e.knife or r in mismatched:

            continue

        if lp is not None:

            assert bf16_within(float(lp[r, 0]), e.logprob, floor=LOGPROB_FLOOR), (r, float(lp[r, 0]), e.logprob)

        if top is not None:

            for z, (t, v) in enumerate(zip(e.top_tokens, e.top_logprobs)):

                assert int(top_tokens[r, z]) == t, (r, z, int(top_tokens[r, z]), t)
                assert bf16_within(float(top_values[r, z]), v, floor=LOGPROB_FLOOR), (r, z, float(top_values[r, z]), v)

        if probs is not None and e.probs is not None:

            slot = int(slot_mapping[r]) if slot_mapping is not None else r

            for t, v in e.probs.items():

                assert bf16_within(float(probs[slot, t]), v), (r, t, float(probs[slot, t]), v)

        checked += 1

    return mismatched, checked


def check_multistep(verification, expected, cu_seqlens, *, logprobs: bool,
                    max_knife_fraction: float = 0.05):

    tokens = verification.tokens.reshape(-1).cpu()
    offsets = verification.offsets.reshape(-1).cpu()
    lp = verification.logprobs.selected.reshape(-1).float().cpu() if logprobs else None
    top = verification.logprobs.top_k if logprobs and verification.logprobs else None
    top_tokens = top.tokens.reshape(-1, top.tokens.size(-1)).cpu() if top is not None else None
    top_values = top.logprobs.reshape(-1, top.logprobs.size(-1)).float().cpu() if top is not None else None

    mismatched = []

    for b, e in enumerate(expected):

        margin = cu_seqlens[b]
        got = [int(t) for t in tokens[margin: margin + int(offsets[b]) + 1]]

        if int(offsets[b]) != e.offset or got != e.tokens:

            mismatched.append(b)

    unexplained = [b for b in mismatched if not expected[b].knife]

    assert not unexplained, [
        (b, int(offsets[b]), expected[b].offset,
         [int(t) for t in tokens[cu_seqlens[b]: cu_seqlens[b] + int(offsets[b]) + 1]], expected[b].tokens)
        for b in unexplained[:6]
    ]

    assert len(mismatched) <= max(1, int(max_knife_fraction * len(expected)))

    for b, e in enumerate(expected):

        if b in mismatched or e.knife or not logprobs:

            continue

        margin = cu_seqlens[b]

        for i, v in enumerate(e.logprobs):

            assert bf16_within(float(lp[margin + i]), v, floor=LOGPROB_FLOOR), (b, i, float(lp[margin + i]), v)

        if top is not None:

            for i, (tt, tv) in enumerate(zip(e.top_tokens, e.top_logprobs)):

                for z, (t, v) in enumerate(zip(tt, tv)):

                    assert int(top_tokens[margin + i, z]) == t, (b, i, z)
                    assert bf16_within(float(top_values[margin + i, z]), v, floor=LOGPROB_FLOOR), (b, i, z, float(top_values[margin + i, z]), v)

    return mismatched


def expected_singular_counts(decode, expected, selection, mismatched, slot_mapping=None, prefill=False):
    """Decode counts a singular call with ``update_counts`` must leave: the oracle's update on every
    row that matches it, and on a knife-edge row (whose token may legitimately differ) the update
    of the token the GPU selected. Every row's counts are compared, also in runs with knife-edge
    rows."""

    tokens = selection.tokens[:, 0].cpu()
    chosen = [SimpleNamespace(token=int(tokens[r]) if r in mismatched else e.token)
              for r, e in enumerate(expected)]

    return oracle.apply_singular_counts(decode, chosen, slot_mapping, prefill=prefill)


def expected_multistep_counts(decode, expected, verification, cu_seqlens, mismatched, slot_mapping=None):
    """Decode counts a verifier call with ``update_counts`` must leave: +1 per emitted token, the
    oracle's tokens for every request that matches it and the GPU's emitted span for a knife-edge
    request, so no request's counts go unchecked."""

    tokens = verification.tokens.reshape(-1).cpu()
    offsets = verification.offsets.reshape(-1).cpu()
    emitted = []

    for b, e in enumerate(expected):

        if b in mismatched:

            m = cu_seqlens[b]
            emitted.append(SimpleNamespace(tokens=[int(t) for t in tokens[m: m + int(offsets[b]) + 1]]))

        else:

            emitted.append(e)

    return oracle.apply_multistep_counts(decode, emitted, slot_mapping)


def load_into(dst, src):
    """Copies every device tensor of a (device) SamplingBuffers from a CPU one of the same layout,
    in place, so that a captured graph sees the new contents at the same addresses."""

    from sonic_sampler.core.flags import Flags

    if isinstance(dst, Flags):

        dst.packed.copy_(src.packed)

    elif dataclasses.is_dataclass(dst):

        for f in dataclasses.fields(dst):

            load_into(getattr(dst, f.name), getattr(src, f.name))

    elif isinstance(dst, torch.Tensor) and dst.device.type == "cuda":

        dst.copy_(src)


def run_verifier(work, *, in_place=False, update_counts=False, logprobs=True, block_size=None,
                 slot_mapping=None, buffers=None, all_greedy=False):

    from bench import to_device
    from sonic_sampler.interface import UnshardedFusedMultistep

    batch = len(work.cu_seqlens) - 1
    buffers = buffers if buffers is not None else to_device(work.buffers, "cuda:0")
    verifier = UnshardedFusedMultistep.initialize(vocab_size=work.vocab, lookahead=work.lookahead,
                                                  batch_size=batch, block_size=block_size,
                                                  max_top_logprobs=work.max_top_logprobs, device="cuda:0")
    drafted = work.drafted.to("cuda:0")

    if work.varlen:

        logits = work.logits.to("cuda:0")
        tokens = drafted
        cu = torch.tensor(work.cu_seqlens, dtype=torch.int32, device="cuda:0")

    else:

        n = work.lookahead + 1
        logits = work.logits.view(batch, n, -1).to("cuda:0")
        tokens = drafted.view(batch, n)
        cu = None

    probs = work.probabilities.to("cuda:0") if work.probabilities is not None else None
    verification = verifier(logits, tokens, buffers, probabilities=probs, update_counts=update_counts,
                            logprobs=logprobs, in_place=in_place, cu_seqlens=cu,
                            slot_mapping=slot_mapping, all_greedy=all_greedy)
    torch.cuda.synchronize()

    return verification, buffers, verifier


def merge_path_logits(rows: int, vocab: int, block: int, seed: int):
    """bf16 logits whose rows take each path of the row merge at tiles = vocab / block (kp = 4 at
    128 tiles): r % 5 == 0 plain spiked values (sampled merge), 1: 60 large values in each of 3
    tiles and 4: 6 in each of 16 tiles (lists merged whole, up to the bound of 16), 2: 8 in each
    of 24 tiles and 3: every logit equal (radix merge)."""

    from bench import spiked_logits

    g = torch.Generator().manual_seed(seed)
    logits = spiked_logits(rows, vocab, seed=seed + 1).float()
    tiles = vocab // block

    for r in range(rows):

        kind = r % 5

        if kind == 3:

            logits[r] = 0.25
            continue

        hot, per = {1: (3, 60), 2: (24, 8), 4: (16, 6)}.get(kind, (0, 0))

        for t in torch.randperm(tiles, generator=g)[:hot].tolist():

            cols = t * block + torch.randperm(block, generator=g)[:per]
            logits[r, cols] = 20.0 + torch.rand(per, generator=g) * 8.0

    return logits.to(torch.bfloat16)
