"""The host population path of SamplingBuffers (reference core/buffer.py:166-764, 1026-1352) on
CPU-resident buffers: request admission, per-iteration updates, weight refresh and staging."""

import torch

from sonic_sampler.core.buffer import SamplingBuffers, TokenCounts, resolve_updates
from sonic_sampler.core.flags import Indicator

BF16 = torch.bfloat16


def bf(v):

    return float(torch.tensor(v).to(BF16))


def admit(buffers, positions):

    encodings = [torch.tensor([3, 3, 7]), torch.tensor([0, 511, 511, 511])]
    buffers.allocate(
        encodings=encodings, multiplicative=[1.2, 1.0], frequency=[0.5, 0.0], presence=[0.25, 0.0],
        biases=[{5: 1.5, 9: -2.0}, None], temperature=[0.7, 1.0], top_k=[20, 128], top_p=[0.9, 1.0],
        min_p=[0.0, 0.05], top_logprobs=[3, 0], positions=positions,
        generator=torch.Generator().manual_seed(1))

    return encodings


def test_allocate_admits_requests_into_slots():

    b = SamplingBuffers.default(size=6, timesteps=3, vocab_size=512, device="cpu")
    b.repetition.counts.decode.fill_(4)
    before = b.weights.gumbel.target.clone()
    admit(b, [1, 4])

    ctx = b.repetition.counts.context
    assert ctx[1, 3] == 2 and ctx[1, 7] == 1 and int(ctx[1].sum()) == 3
    assert ctx[4, 0] == 1 and ctx[4, 511] == 3 and int(ctx[4].sum()) == 4
    assert int(b.repetition.counts.decode[1].abs().sum()) == 0 and int(b.repetition.counts.decode[4].abs().sum()) == 0
    assert int(b.repetition.counts.decode[0, 0]) == 4          # other slots untouched

    assert float(b.temperature[1]) == bf(0.7) and float(b.top_p[1]) == bf(0.9) and int(b.top_k[1]) == 20
    assert float(b.min_p[4]) == bf(0.05) and int(b.top_logprobs[1]) == 3
    assert float(b.repetition.multiplicative[1]) == bf(1.2) and float(b.repetition.frequency[1]) == 0.5
    assert float(b.bias[1, 5]) == 1.5 and float(b.bias[1, 9]) == -2.0 and int((b.bias[1] != 0).sum()) == 2

    # indicators follow the parameters: slot 1 has penalties, bias, temperature, top-k / top-p
    t1 = Indicator(int(b.flags.indicators.target[1]))
    for bit in (Indicator.MULTIPLICATIVE, Indicator.FREQUENCY, Indicator.PRESENCE, Indicator.BIAS,
                Indicator.TEMPERATURE, Indicator.TOP_K, Indicator.TOP_P, Indicator.TOP_K_LOGPROBS):
        assert bit in t1
    assert int(b.flags.packed[1, 0]) == int(t1)

    # stochastic slots get prefill noise at step 0 (other steps and slots keep theirs)
    assert not torch.equal(b.weights.gumbel.target[1, 0], before[1, 0])
    assert torch.equal(b.weights.gumbel.target[1, 1:], before[1, 1:])
    assert torch.equal(b.weights.gumbel.target[0], before[0])


def test_update_refreshes_parameters_and_counts_in_order():

    b = SamplingBuffers.default(size=3, timesteps=2, vocab_size=64, device="cpu")
    counts = [(torch.full((64,), 2, dtype=torch.int32), torch.arange(64, dtype=torch.int32))] * 3
    targets = [None, torch.zeros(2, 64, dtype=BF16), None]
    b.update(counts=counts, target_gumbel=targets, multiplicative=[1.0, 1.0, 1.0], frequency=[0.0, 0.3, 0.0],
             presence=[0.0, 0.0, 0.0], biases=[None, None, None], temperature=[1.0, 0.5, 1.0],
             top_k=[1, 50, 1], top_p=[1.0, 1.0, 1.0], min_p=[0.0, 0.0, 0.0], top_logprobs=[0, 0, 0])
    assert Indicator.GREEDY in Indicator(int(b.flags.indicators.target[0]))
    assert int(b.top_k[1]) == 50 and float(b.temperature[1]) == 0.5
    assert torch.equal(b.repetition.counts.decode[1], torch.arange(64, dtype=torch.int32))
    assert int(b.repetition.counts.context[0, 7]) == 2
    assert torch.equal(b.weights.gumbel.target[1], torch.zeros(2, 64, dtype=BF16))   # the drafter's noise


def test_resolve_updates_shapes():

    g = torch.Generator()
    assert resolve_updates(4, g) == [(None, g, (True, True), False)]
    assert resolve_updates(4, None, prefill=True) == [(None, None, (True, True), True)]
    per = resolve_updates(4, [g, g], selectors=[(True, False), (False, True)], positions=[2, 0], prefill=[True, False])
    assert per == [(2, g, (True, False), True), (0, g, (False, True), False)]
    assert [r[0] for r in resolve_updates(3, g, selectors=[(True, True)] * 3)] == [0, 1, 2]


def test_token_counts_populate_histograms_prompts():

    c = TokenCounts.zeros(4, 1, 16)
    c.allocate([torch.tensor([1, 1, 15]), torch.tensor([2])], positions=[3, 0])
    assert c.context[3].tolist()[1] == 2 and c.context[3].tolist()[15] == 1 and int(c.context[3].sum()) == 3
    assert c.context[0].tolist()[2] == 1 and int(c.context[1].sum()) == 0


def test_step_weights_stages_draft_noise_for_stochastic_drafters():

    b = SamplingBuffers.default(size=4, timesteps=2, vocab_size=512, device="cpu")
    admit(b, [1, 2])   # slot 1 stochastic (top-k 20, temperature), slot 2 stochastic (min-p)
    draft = b.weights.gumbel.draft.clone()
    b.step_weights(positions=[1, 2], indices=torch.tensor([1, 2]), generator=torch.Generator().manual_seed(3))
    # the verifier's noise of a stochastic drafter is the drafter's noise of the last iteration
    assert torch.equal(b.weights.gumbel.target[1], draft[1])
    # and the drafter's noise is redrawn
    assert not torch.equal(b.weights.gumbel.draft[1], draft[1])
