"""The host population path of SamplingBuffers (reference core/buffer.py:166-764, 1026-1352) on
CPU-resident buffers: request admission, per-iteration updates, weight refresh and staging."""

import pytest
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


def test_update_takes_carried_noise_on_decode_rows_with_per_request_prefill():
    """With ``prefill`` given per request (the just-in-time guide's form), the carried drafter noise
    of each decode row replaces its verifier noise; a prefill row keeps what it drew."""

    b = SamplingBuffers.default(size=3, timesteps=2, vocab_size=64, device="cpu")
    counts = [(torch.zeros(64, dtype=torch.int32), torch.zeros(64, dtype=torch.int32))] * 3
    carried = [torch.full((2, 64), -1.5, dtype=BF16), torch.full((2, 64), -2.5, dtype=BF16), None]
    b.update(counts=counts, target_gumbel=carried, multiplicative=[1.0] * 3, frequency=[0.0] * 3,
             presence=[0.0] * 3, biases=[None] * 3, temperature=[0.9] * 3, top_k=[50] * 3, top_p=[1.0] * 3,
             min_p=[0.0] * 3, top_logprobs=[0] * 3, prefill=[False, True, False],
             generator=[torch.Generator().manual_seed(i) for i in range(3)])
    assert torch.equal(b.weights.gumbel.target[0], carried[0])
    assert not torch.equal(b.weights.gumbel.target[1], carried[1])
    assert bool(torch.isfinite(b.weights.gumbel.target[2].float()).all())


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


def test_step_weights_redraws_noise_of_positions_on_host_buffers():
    """Without device rows to stage from (``indices=None``) step_weights only redraws: the
    drafter's noise of stochastic drafters, and the acceptance uniforms, of `positions` only."""

    b = SamplingBuffers.default(size=4, timesteps=2, vocab_size=512, device="cpu")
    admit(b, [1, 2])   # slot 1 stochastic (top-k 20, temperature), slot 2 stochastic (min-p)
    draft = b.weights.gumbel.draft.clone()
    uniform = b.weights.uniform.clone()
    b.step_weights(positions=[1], generator=torch.Generator().manual_seed(3))
    assert not torch.equal(b.weights.gumbel.draft[1], draft[1])
    assert not torch.equal(b.weights.uniform[1], uniform[1])
    assert torch.equal(b.weights.gumbel.draft[2], draft[2])
    assert torch.equal(b.weights.uniform[2], uniform[2])


def test_noise_staging_needs_device_buffers():
    """Staging the drafter's noise is the ss_indexed_copy kernel's job: host-resident planes are
    refused rather than copied by a host fallback."""

    b = SamplingBuffers.default(size=4, timesteps=2, vocab_size=512, device="cpu")
    admit(b, [1, 2])

    with pytest.raises(RuntimeError, match="on a GPU"):

        b.step_weights(positions=[1, 2], indices=torch.tensor([1, 2]), generator=torch.Generator().manual_seed(3))

