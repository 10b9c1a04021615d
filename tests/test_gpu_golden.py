"""The HIP path against the committed golden fixtures (tests/golden/*.json).

Each case's inputs are regenerated from the fixture's parameters (under the fixtures' CPU
settings, in a child process) and checked against its input digests, then run through the
library. The outputs must meet the stored ones (no oracle call here): tokens, offsets and
top-logprob ids exactly, logprobs and probabilities within the bf16 output tolerance of the parity
tests, the per-row top-128 ids exactly, and the decode counts after the update exactly.
"""

import json

from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from helpers import check_multistep, check_singular, run_verifier
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):

    return json.loads((GOLDEN / f"{name}.json").read_text())


def rows_of(case):
    """Stored row records in the shape check_singular reads."""

    return [SimpleNamespace(token=r["token"], greedy=r["greedy"], knife=r["knife"], logprob=r["logprob"],
                            top_tokens=r["top_tokens"], top_logprobs=r["top_logprobs"],
                            probs=None if r["probs"] is None else {int(k): v for k, v in r["probs"].items()})
            for r in case["rows"]]


def requests_of(case):

    return [SimpleNamespace(**{k: v for k, v in r.items()}) for r in case["requests"]]


def inputs(name):
    """The case's inputs as the fixture was made from them, checked against its digests."""

    from golden import make_fixtures as mf

    case = load(name)
    w = mf.fixture_inputs(name)
    got = {"logits": mf.digest(w.logits), **mf.state_digests(w.buffers, name)}
    got.update({attr: mf.digest(getattr(w, attr)) for attr in mf.EXTRA[name]})
    assert got == case["inputs"], f"{name}: regenerated inputs differ from the fixture's"

    return case, w


def test_singular_fixture():

    from bench import to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    case, w = inputs("singular")
    batch, vocab = w.logits.shape
    print(f"golden singular: B={batch} V={vocab}", flush=True)
    buffers = to_device(w.buffers, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch, max_top_logprobs=5, device=DEV)
    selection = sampler.autoregressive(w.logits.to(DEV), buffers, update_counts=True, logprobs=True)
    torch.cuda.synchronize()

    expected = rows_of(case)
    check_singular(selection, expected, logprobs=True, max_knife_fraction=0.0)

    counts = oracle.apply_singular_counts(w.buffers.repetition.counts.decode.clone(), expected, None, prefill=False)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_drafting_fixture():

    from bench import to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    case, w = inputs("drafting")
    rows = w.logits.size(0)
    slots = w.buffers.layout.rows
    print(f"golden drafting: rows={rows} slots={slots} V_d={w.vocab} V_t={w.target_vocab}", flush=True)
    buffers = to_device(w.buffers, DEV)
    # 1024-column tiles: the 2000-column draft vocabulary must span more than one tile
    sampler = UnshardedFusedSingular.initialize(vocab_size=w.vocab, batch_size=rows, lookahead=4,
                                                max_top_logprobs=5, block_size=1024, device=DEV)
    probs = torch.zeros(slots, w.target_vocab, dtype=torch.bfloat16, device=DEV)
    selection = sampler.drafting(w.logits.to(DEV), buffers, timestep=w.timestep, tokens=w.tokens.to(DEV),
                                 probabilities=probs, slot_mapping=w.slot_mapping.to(DEV),
                                 d2t_mapping=w.d2t.to(DEV), target_vocab=w.target_vocab, in_place=True)
    torch.cuda.synchronize()

    check_singular(selection, rows_of(case), logprobs=False, probabilities=probs, slot_mapping=w.slot_mapping,
                   max_knife_fraction=0.0)


def test_multistep_fixture():

    case, w = inputs("multistep")
    print(f"golden multistep: rows={w.logits.size(0)} requests={len(w.cu_seqlens) - 1}", flush=True)
    assert list(w.cu_seqlens) == case["cu_seqlens"]
    verification, buffers, verifier = run_verifier(w, update_counts=True)

    expected = requests_of(case)
    check_multistep(verification, expected, w.cu_seqlens, logprobs=True, max_knife_fraction=0.0)
    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert indices[w.cu_seqlens[b] + i].tolist() == idx, (b, i)

    counts = oracle.apply_multistep_counts(w.buffers.repetition.counts.decode.clone(), expected, None)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_topk_fixture():

    from golden import make_fixtures as mf
    from sonic_sampler.interface import UnshardedBoundedTopK

    case = load("topk")
    x = mf.fixture_inputs("topk")
    assert mf.digest(x) == case["inputs"]["logits"]
    rows, vocab, k = case["params"]["rows"], case["params"]["vocab"], case["params"]["k"]
    print(f"golden top-k: rows={rows} V={vocab} k={k}", flush=True)
    topk = UnshardedBoundedTopK.initialize(vocab_size=vocab, batch_size=rows, k=k, device=DEV)
    values, indices = topk(x.to(DEV))
    torch.cuda.synchronize()

    assert indices.cpu().tolist() == case["indices"]
    assert values.cpu().tolist() == case["values"]
