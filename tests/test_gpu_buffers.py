"""ss_indexed_copy (the reference's indexed_copy, ops/copy.py:21-127) and the GPU weight step of
SamplingBuffers against torch's indexing."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BF16 = torch.bfloat16


@pytest.mark.parametrize("vocab", [4096, 1001])
def test_indexed_copy_stages_stochastic_slots(vocab):
    """16-byte rows (V = 4096) and rows of an odd width (3 x 1001 elements, element copies);
    greedy slots keep their target rows and indices outside the slots are skipped."""

    from sonic_sampler import _native

    slots, steps = 10, 3
    g = torch.Generator().manual_seed(vocab)
    draft = torch.randn(slots, steps, vocab, generator=g).to(BF16)
    target = torch.randn(slots, steps, vocab, generator=g).to(BF16)
    indicators = torch.tensor([0x40 if i % 3 == 0 else 0x80 for i in range(slots)], dtype=torch.int32)
    indices = torch.tensor([7, 3, 0, 9, 5, 12, -1], dtype=torch.int64)
    expected = target.clone()

    for i in indices.tolist():

        if 0 <= i < slots and not indicators[i] & 0x40:

            expected[i] = draft[i]

    got = target.to(DEV)
    print(f"indexed copy V={vocab}", flush=True)
    _native.indexed_copy(draft.to(DEV), got, indices.to(DEV), indicators.to(torch.uint16).to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), expected)


def test_step_weights_on_device_buffers():

    from bench import to_device
    from sonic_sampler.core.buffer import SamplingBuffers

    host = SamplingBuffers.random(size=8, timesteps=3, vocab_size=2048, device="cpu", seed=4)
    b = to_device(host, DEV)
    positions = [6, 1, 3]
    draft = b.weights.gumbel.draft.clone()
    target = b.weights.gumbel.target.clone()
    print("step_weights on device buffers", flush=True)
    b.step_weights(positions=positions, indices=torch.tensor(positions, device=DEV),
                   generator=torch.Generator(DEV).manual_seed(1))
    torch.cuda.synchronize()
    scoped = host.flags.indicators

    for i in range(8):

        if i not in positions:

            assert torch.equal(b.weights.gumbel.target[i], target[i])
            assert torch.equal(b.weights.gumbel.draft[i], draft[i])

        elif int(scoped.draft[i]) & 0x40 == 0:

            assert torch.equal(b.weights.gumbel.target[i], draft[i])


def test_autotune_measures_a_small_table(tmp_path):

    from sonic_sampler.interface.autotune import autotune, measure_kind
    from sonic_sampler.interface.dispatch import DispatchSummary

    print("autotune: 2 vocabularies x 2 batches x 4 call kinds", flush=True)
    summary = autotune([8192, 32768], [1, 16], measure=lambda *key: measure_kind(*key, steps=5, warmup=1),
                       log=lambda line: print(line, flush=True))
    path = tmp_path / "table.toml"
    summary.save(path)
    back = DispatchSummary.read(path)
    assert back.vocab.get(32768).batch.get(16).best.block_n in (1024, 2048, 4096, 8192, 16384)
    assert len(back.vocab.get(8192).batch.get(1).config) == 1


def test_flags_update_reaches_the_device_words():
    """Flags.update at scattered and at leading positions, on a copy stream: the device words the
    kernels read equal the readable lists afterwards, and all_greedy follows them."""

    from sonic_sampler.core.flags import Flags, Indicator, ScopedIndicators

    greedy, stochastic = Indicator.GREEDY | Indicator.GRAMMAR, Indicator.TEMPERATURE | Indicator.TOP_P
    flags = Flags.from_values(16, 4, greedy, device="cuda:0")
    stream = torch.cuda.Stream()
    expect = lambda: torch.tensor([[int(t), int(d)] for t, d in zip(flags.indicators.target,
                                                                     flags.indicators.draft)], dtype=torch.int32)

    assert flags.all_greedy
    flags.update(ScopedIndicators.from_values(size=3, timesteps=4, target=[stochastic] * 3,
                                              draft=[greedy, stochastic, greedy]), positions=[11, 2, 7], stream=stream)
    stream.synchronize()
    assert torch.equal(flags.packed.cpu().to(torch.int32), expect())
    assert not flags.all_greedy

    flags.update(ScopedIndicators.from_values(size=2, timesteps=4, target=[greedy] * 2), positions=None, stream=stream)
    stream.synchronize()
    assert torch.equal(flags.packed.cpu().to(torch.int32), expect())
    assert flags.packed.stride() == (1, 16)
