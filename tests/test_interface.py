"""Host-side surface on the CPU: indicator derivation, buffer layouts, dispatch resolution and the
functional entry points' argument errors (raised before any device work). Each block cites the
reference module whose behaviour it checks (the reference ships no tests of its own)."""

from __future__ import annotations

import pytest
import torch

from sonic_sampler.core.flags import Flags, Indicator, SamplingMode, ScopedIndicators
from sonic_sampler.core.buffer import SamplingBuffers
from sonic_sampler.interface.base import TwoStageTiling, resolve_dispatch
from sonic_sampler.interface.dispatch import DispatchSummary
from sonic_sampler.ops.base import MAX_K, next_power_of_2


# ------------------------------------------------------------------------------------------------
# Indicators (reference core/flags.py:150-184)
# ------------------------------------------------------------------------------------------------

def test_greedy_is_top_k_one_and_masks_stochastic_bits():

    bits = Indicator.from_params(temperature=0.7, top_k=1, top_p=0.9, min_p=0.1, top_k_logprobs=5,
                                 greedy_draft=True)

    assert Indicator.GREEDY in bits
    assert Indicator.TEMPERATURE in bits
    for masked in (Indicator.TOP_K, Indicator.TOP_P, Indicator.MIN_P, Indicator.TOP_K_LOGPROBS,
                   Indicator.STOCHASTIC_VERIFY_GREEDY_DRAFT):
        assert masked not in bits


@pytest.mark.parametrize("top_k, expected", [(0, False), (1, False), (2, True), (127, True), (128, False),
                                             (1000, False)])
def test_top_k_bit_only_strictly_inside_the_bound(top_k, expected):

    assert (Indicator.TOP_K in Indicator.from_params(top_k=top_k)) is expected


@pytest.mark.parametrize("field, value, bit", [
    ("multiplicative", 1.1, Indicator.MULTIPLICATIVE),
    ("frequency", 0.2, Indicator.FREQUENCY),
    ("presence", -0.3, Indicator.PRESENCE),
    ("temperature", 0.5, Indicator.TEMPERATURE),
    ("top_p", 0.9, Indicator.TOP_P),
    ("min_p", 0.05, Indicator.MIN_P),
    ("top_k_logprobs", 5, Indicator.TOP_K_LOGPROBS),
])
def test_each_parameter_sets_its_bit(field, value, bit):

    assert bit in Indicator.from_params(**{field: value})
    assert Indicator.from_params() & bit == 0


def test_neutral_parameters_give_no_bits():

    assert int(Indicator.from_params()) == 0
    assert int(Indicator.from_params(top_p=1.0, min_p=0.0, top_k=MAX_K)) == 0


def test_greedy_resolution_and_modes():

    full = Indicator.maximal()

    assert full.greedy() & Indicator.stochastic() == 0
    assert Indicator.GREEDY in full.greedy()
    assert full.resolve(SamplingMode.MINIMAL) == Indicator.GREEDY
    assert Indicator.GRAMMAR not in full.resolve(SamplingMode.NON_GRAMMAR)
    assert Indicator.GREEDY not in full
    assert int(Indicator.all()) == 0xFFF


def test_flags_pack_target_and_draft_contiguously():

    target = [Indicator.from_params(top_k=1), Indicator.from_params(temperature=0.5), Indicator.GRAMMAR]
    draft = [Indicator.GREEDY, Indicator.GREEDY, Indicator.BIAS]
    flags = Flags.from_scoped(ScopedIndicators.from_values(3, 4, target, draft), device="cpu")

    assert flags.packed.shape == (3, 2)
    assert flags.packed.stride() == (1, 3)
    assert flags.target.is_contiguous() and flags.draft.is_contiguous()
    assert flags.target.tolist() == [int(t) for t in target]
    assert flags.draft.tolist() == [int(d) for d in draft]
    assert not flags.all_greedy


# ------------------------------------------------------------------------------------------------
# Buffers (reference core/buffer.py:784-817, :938-986)
# ------------------------------------------------------------------------------------------------

def test_default_buffers_are_neutral():

    size, steps, vocab = 3, 4, 1000
    buffers = SamplingBuffers.default(size, steps, vocab, device="cpu", noise=False)

    assert buffers.grammar.shape == (size, steps, (vocab + 31) // 32)
    assert buffers.grammar.dtype == torch.uint32
    assert torch.all(buffers.grammar.view(torch.int32) == -1)       # every token allowed
    assert buffers.bias.shape == (size, vocab) and not buffers.bias.float().any()
    assert torch.all(buffers.temperature.float() == 1.0)
    assert torch.all(buffers.top_k == MAX_K)
    assert torch.all(buffers.top_p.float() == 1.0)
    assert not buffers.min_p.float().any()
    counts = buffers.repetition.counts
    assert counts.context.shape == counts.decode.shape == (size, vocab)
    assert counts.decode.dtype == torch.int32
    assert buffers.weights.gumbel.target.shape == (size, steps, vocab)
    assert buffers.flags.packed.shape == (size, 2)


def test_random_buffers_are_reproducible_and_honour_indicators():

    a = SamplingBuffers.random(4, 2, 512, device="cpu", seed=5)
    b = SamplingBuffers.random(4, 2, 512, device="cpu", seed=5)

    assert torch.equal(a.flags.packed, b.flags.packed)
    assert torch.equal(a.temperature, b.temperature)
    assert torch.equal(a.repetition.counts.decode, b.repetition.counts.decode)

    for row, word in enumerate(a.flags.target.tolist()):

        bits = Indicator(word)
        if Indicator.TEMPERATURE not in bits:
            assert float(a.temperature[row]) == 1.0
        if Indicator.MIN_P not in bits:
            assert float(a.min_p[row]) == 0.0


# ------------------------------------------------------------------------------------------------
# Dispatch and tiling (reference interface/dispatch.py:105-268, interface/base.py:155-276)
# ------------------------------------------------------------------------------------------------

def test_dispatch_table_for_gfx950():

    table = DispatchSummary.load(k=MAX_K, arch="gfx950")

    assert table is not None
    # a vocabulary bucket's block_n is its smallest width (the scratchpad is sized for it); a
    # launch takes the width of the bucket of its row count
    assert table.vocab.get(size=128256).block_n == 2048
    assert table.vocab.get(size=32000).block_n == 1024
    assert table.vocab.get(size=128256).batch.get(size=64).best.block_n == 4096     # config 1
    assert table.vocab.get(size=128256).batch.get(size=2048).best.block_n == 8192


def test_call_kind_tables_for_gfx950():
    """The verification and the drafting step read tables of their own; a kind without a bucket
    for the vocabulary (drafting is measured for draft vocabularies only) takes the shared one."""

    multistep = DispatchSummary.load(k=MAX_K, arch="gfx950", kind="multistep")
    drafting = DispatchSummary.load(k=MAX_K, arch="gfx950", kind="drafting")

    assert DispatchSummary.load(k=MAX_K, arch="gfx950", kind="absent") is None
    assert multistep.vocab.get(size=128256).batch.get(size=294).best.block_n == 16384   # config 3
    assert multistep.vocab.get(size=151936).batch.get(size=640).best.block_n == 16384   # config 2
    assert drafting.vocab.get(size=32000).batch.get(size=256).best.block_n == 8192      # config 4
    assert drafting.vocab.get(size=128256) is None
    topk = DispatchSummary.load(k=MAX_K, arch="gfx950", kind="topk")
    assert topk.vocab.get(size=32000).batch.get(size=8).best.block_n == 1024             # config 0

    shared, _ = resolve_dispatch(MAX_K, 128256, None, "gfx950")
    own, _ = resolve_dispatch(MAX_K, 128256, None, "gfx950", kind="multistep")
    fallback, _ = resolve_dispatch(MAX_K, 128256, None, "gfx950", kind="drafting")
    assert own.batch.get(size=294).best.block_n == 16384
    assert fallback.batch.get(size=294).best.block_n == shared.batch.get(size=294).best.block_n == 8192

    # buffers shared by the decode and drafting steps hold the lists of the smaller width of the two
    tiling, _, _ = TwoStageTiling.factory(vocab_size=32000, batch_size=256, arch="gfx950", device="cpu",
                                          kinds=(None, "drafting"))
    assert tiling.block_n == min(tiling.dispatch.block_n, tiling.kind_dispatch["drafting"].block_n) == 1024
    assert tiling.scratchpad.shape == (256, 32 * MAX_K)
    assert tiling.tuning(256)[2] == 4096
    assert tiling.tuning(256, kind="drafting")[2] == 8192
    assert tiling.tuning(256, kind="topk")[2] == 4096   # no table of that kind was resolved


@pytest.mark.parametrize("k, block, message", [
    (256, None, "maximum supported top-k"),
    (48, None, "power of 2"),
    (128, 3000, "block_size"),
])
def test_dispatch_errors(k, block, message):

    with pytest.raises(ValueError, match=message):

        resolve_dispatch(k, 32000, block, "gfx950")


def test_tiling_buffers():

    tiling, values, indices = TwoStageTiling.factory(vocab_size=128256, batch_size=8, lookahead=3,
                                                     arch="gfx950", device="cpu")

    # sized for the bucket's smallest width (2048: 63 tiles); 32 rows launch at 4096
    assert tiling.block_n == 2048
    assert tiling.vocabulary.blocks == 63
    assert tiling.scratchpad.shape == (8 * 4, 63 * MAX_K)
    assert tiling.tuning(32)[2] == 4096
    assert tiling.scratchpad.dtype == torch.uint32
    assert values.shape == indices.shape == (32, MAX_K)


@pytest.mark.parametrize("vocab", [2049, 3000, 4096, 5000, 8192, 9000, 20000])
def test_launch_width_never_leaves_a_single_tile(vocab):
    """A vocabulary bucket's tuned widths are measured on its larger sizes; at every batch size the
    launch width must still split the vocabulary into at least two tiles, and never into more
    than the scratchpad holds (the top-k table tunes V = 3000 at 4 rows to 4096: the buffers'
    2048 is used)."""

    for kinds in ((None,), ("topk",)):

        tiling, _, _ = TwoStageTiling.factory(vocab_size=vocab, batch_size=8, arch="gfx950", device="cpu",
                                              kinds=kinds)

        for rows in (1, 2, 4, 8, 16, 64, 256, 1024):

            block_n = tiling.tuning(rows)[2]
            tiles = -(-vocab // block_n)

            assert 2 <= tiles <= tiling.vocabulary.blocks, (kinds, rows, block_n)

        if vocab == 3000 and kinds == ("topk",):

            assert tiling.tuning(4)[2] == tiling.block_n == 2048


def test_tuning_is_kept_per_instance_and_follows_its_tables():
    """The lookup without an explicit strategy or tuning is computed once per row count, equal to
    a fresh one, and recomputed when the instance's tables are replaced."""

    from sonic_sampler.interface import UnshardedFusedMultistep

    tiling, _, _ = TwoStageTiling.factory(vocab_size=128256, batch_size=64, arch="gfx950", device="cpu")
    first = tiling.tuning(64)

    assert tiling.tuning(64) is first
    assert tiling._tuning(64, None, None, None)[2] == first[2]

    tiling.dispatch = None

    assert tiling.tuning(64) is not first and tiling.tuning(64)[2] == tiling.block_n

    verifier = UnshardedFusedMultistep.initialize(vocab_size=128256, lookahead=3, batch_size=16, device="cpu")
    config, _, block_n = verifier.tuning(64)

    assert verifier.tuning(64)[0] is config and config.third == 4 and block_n == verifier.tuning(64)[2]


def test_single_tile_vocabulary_is_rejected():

    with pytest.raises(ValueError, match="greater than 1"):

        TwoStageTiling.factory(vocab_size=1000, block_size=1024, device="cpu")


def test_next_power_of_2():

    assert [next_power_of_2(n) for n in (1, 2, 3, 5, 128, 129)] == [1, 2, 4, 8, 128, 256]


# ------------------------------------------------------------------------------------------------
# Functional argument errors (reference interface/functional/*.py ValueError conditions)
# ------------------------------------------------------------------------------------------------

def test_fused_singular_argument_errors():

    from sonic_sampler.interface.functional.singular import fused_singular

    logits = torch.zeros(2, 8192, dtype=torch.bfloat16)
    flags = torch.zeros(2, dtype=torch.uint16)

    with pytest.raises(ValueError, match="bfloat16"):
        fused_singular(logits.float(), flags, block_n=1024)
    with pytest.raises(ValueError):
        fused_singular(logits, flags, block_n=1000)
    with pytest.raises(ValueError, match="top logprobs"):
        fused_singular(logits, flags, block_n=1024, max_top_logprobs=129)
    with pytest.raises(ValueError, match="local rank"):
        fused_singular(logits, flags, block_n=1024, world_size=2, local_rank=2)
    with pytest.raises(ValueError, match="shard size"):
        fused_singular(logits, flags, block_n=1024, world_size=2, shard_size=4096)
    with pytest.raises(ValueError, match="stage"):
        fused_singular(logits, flags, block_n=1024, stage="merge")
    with pytest.raises(ValueError):
        fused_singular(logits, flags, block_n=1024, update_counts=True)   # counts required


def test_fused_multistep_layout_errors():

    from sonic_sampler.interface.functional.multistep import fused_multistep

    flags = torch.zeros(2, dtype=torch.uint16)
    drafted = torch.zeros(2, 5, dtype=torch.int32)

    with pytest.raises(ValueError, match="lookahead"):
        fused_multistep(torch.zeros(10, 8192, dtype=torch.bfloat16), flags, drafted, block_n=1024)
    with pytest.raises(ValueError, match="multiple"):
        fused_multistep(torch.zeros(11, 8192, dtype=torch.bfloat16), flags, drafted, block_n=1024, lookahead=4)
    with pytest.raises(ValueError, match="varlen"):
        fused_multistep(torch.zeros(2, 5, 8192, dtype=torch.bfloat16), flags, drafted, block_n=1024,
                        cu_seqlens=torch.tensor([0, 5, 10], dtype=torch.int32))
    with pytest.raises(ValueError, match="63"):
        fused_multistep(torch.zeros(2, 65, 8192, dtype=torch.bfloat16), flags, drafted, block_n=1024)


def test_autotune_ranks_widths_and_round_trips(tmp_path):
    """The table the autotune harness writes holds, per bucket, the width with the smallest worst
    slowdown over the call kinds (never one that leaves a single tile; a kind that has no call of
    the bucket's size is left out), and reads back through DispatchSummary."""

    from sonic_sampler.interface.autotune import autotune
    from sonic_sampler.interface.dispatch import DispatchSummary

    best = {8192: 1024, 131072: 4096}
    seen = []

    def measure(kind, v, b, w):

        seen.append((kind, v, b, w))

        if kind == "multistep" and b < 2:

            return None

        return abs(w - (8192 if b >= 256 else best[v])) + 1.0

    summary = autotune([8192, 131072], [1, 64, 512], measure=measure, kinds=("singular", "multistep", "topk"),
                       arch="gfx950")
    path = tmp_path / "gfx950_k128.toml"
    summary.save(path)
    back = DispatchSummary.read(path)

    assert sorted(w for kind, v, b, w in seen if (kind, v, b) == ("topk", 8192, 1)) == [1024, 2048, 4096]
    assert {kind for kind, *_ in seen} == {"singular", "multistep", "topk"}
    assert [(c.priority, c.block_n) for c in back.vocab.get(8192).batch.get(1).config] == [(0, 1024)]
    assert back.vocab.get(131072).batch.get(64).best.block_n == 4096
    assert back.vocab.get(131072).batch.get(300).best.block_n == 8192
    assert back.vocab.get(131072).block_n == 4096   # the scratchpad is sized for the smallest width

    # a wider width within the tolerance of the best score wins
    times = {1024: 10.0, 2048: 10.1, 4096: 11.0, 8192: 12.0}
    near = autotune([32768], [1], widths=times, measure=lambda kind, v, b, w: times[w])
    assert near.vocab.get(32768).batch.get(1).best.block_n == 2048

    # the worst slowdown over the kinds decides: 4096 is 5% behind on one kind, 1024 2x on another
    split = {"singular": {1024: 10.0, 2048: 11.0, 4096: 10.5, 8192: 13.0},
             "multistep": {1024: 20.0, 2048: 12.0, 4096: 10.0, 8192: 10.2},
             "topk": {1024: 9.0, 2048: 9.5, 4096: 9.2, 8192: 9.9}}
    mixed = autotune([32768], [8], widths=split["singular"], measure=lambda kind, v, b, w: split[kind][w],
                     kinds=split)
    assert mixed.vocab.get(32768).batch.get(8).best.block_n == 4096


def test_autotune_writes_a_table_per_kind_from_a_log(tmp_path):
    """`--from-log` scores an earlier run's times again: one table per kind, the shared one for
    the decode step, buckets where a kind has no call left out."""

    from sonic_sampler.interface.autotune import main, parse_log, table_path
    from sonic_sampler.interface.dispatch import DispatchSummary

    log = tmp_path / "autotune.log"
    log.write_text("\n".join([
        "noise from the runtime",
        "vocab 32768 batch 1: 2048 | singular 1024:10.00 2048:10.10 4096:11.00 8192:12.00",
        "vocab 32768 batch 8: 8192 | singular 1024:10.00 2048:11.00 4096:10.50 8192:13.00 | "
        "multistep 1024:20.00 2048:12.00 4096:10.00 8192:10.10",
    ]) + "\n")

    times = parse_log(log.read_text().splitlines())
    assert times[("multistep", 32768, 8, 8192)] == 10.1
    assert ("multistep", 32768, 1, 1024) not in times

    out = str(tmp_path / "gfx950_k128.toml")
    assert table_path(out, "singular") == out
    assert table_path(out, "multistep") == str(tmp_path / "gfx950_k128_multistep.toml")

    assert main(["--out", out, "--vocab", "32768", "--batch", "1,8", "--widths", "1024,2048,4096,8192",
                 "--kinds", "singular,multistep", "--from-log", str(log)]) == 0
    shared = DispatchSummary.read(out)
    multistep = DispatchSummary.read(table_path(out, "multistep"))

    assert [b.size for b in shared.vocab.get(32768).batch] == [1, 8]
    assert shared.vocab.get(32768).batch.get(1).best.block_n == 2048
    assert shared.vocab.get(32768).batch.get(8).best.block_n == 1024
    assert [b.size for b in multistep.vocab.get(32768).batch] == [8]     # no one-row verification
    assert multistep.vocab.get(32768).batch.get(8).best.block_n == 8192


def test_all_greedy_reads_the_mirror_the_lists_are_kept_in():
    """all_greedy equals the lists' own test for uniform, mixed and updated indicator sets."""

    from sonic_sampler.core.flags import Flags, Indicator, ScopedIndicators

    greedy, stochastic = Indicator.GREEDY | Indicator.GRAMMAR, Indicator.TEMPERATURE

    for target, draft in ((greedy, greedy), (greedy, stochastic), (stochastic, greedy),
                          ([greedy] * 7 + [stochastic], None), ([stochastic] + [greedy] * 7, None)):

        flags = Flags.from_values(8, 3, target, draft, device="cpu")
        lists = flags.indicators.greedy_target and flags.indicators.greedy_draft

        assert flags.all_greedy == lists, (target, draft)

    flags = Flags.from_values(8, 3, greedy, device="cpu")
    assert flags.all_greedy
    flags.update(ScopedIndicators.from_values(size=1, timesteps=3, target=[stochastic]), positions=[5])
    assert not flags.all_greedy and not flags.indicators.greedy_target
    flags.update(ScopedIndicators.from_values(size=1, timesteps=3, target=[greedy]), positions=[5])
    assert flags.all_greedy
    assert flags.subset([0, 1, 2], torch.tensor([0, 1, 2])).all_greedy
