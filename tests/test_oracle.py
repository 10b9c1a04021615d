"""Pins of the CPU oracle (no GPU): known-answer vectors, closed forms, brute force, invariants.

Each test is chosen so that a plausible restatement mistake (a dropped processor, a wrong rounding
point, a flipped comparison, a wrong tie order, an off-by-one in the acceptance chain) fails it.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import philox, topk
from oracle import sampler as oracle

BF16 = torch.bfloat16
I32 = torch.int32


# ------------------------------------------------------------------------------------------------
# Philox4x32-10: Random123 known-answer vectors (kat_vectors, philox4x32_10)
# ------------------------------------------------------------------------------------------------

KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", KAT)
def test_philox_known_answers(counter, key, expected):

    out = philox.philox4x32_10(np.array(counter, dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert tuple(int(x) for x in out) == expected


def test_noise_words_layout():

    words = philox.noise_words(seed=(5 << 32) | 9, offset=3, slots=2, steps=2, vocab=3)
    direct = philox.philox4x32_10(np.array([2, 1, 1, 3], dtype=np.uint32), np.array([9, 5], dtype=np.uint32))
    assert int(words[1, 1, 2]) == int(direct[0])


def test_bf16_round_matches_torch():

    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 100
    x[:4] = [0.0, -0.0, 1.00390625, 1.01171875]  # exact ties round to even
    assert np.array_equal(philox.bf16_round(x), torch.from_numpy(x).to(BF16).float().numpy())


def test_gumbel_transform_statistics():

    w = philox.gumbel_from_words(philox.noise_words(1, 0, 1, 1, 200000))[0, 0]
    # log(E), E ~ Exp(1): mean -gamma_EulerMascheroni, variance pi^2 / 6
    assert abs(w.mean() + 0.5772156649) < 0.01
    assert abs(w.var() - math.pi ** 2 / 6) < 0.03
    assert np.all(np.isfinite(w))


# ------------------------------------------------------------------------------------------------
# Bounded top-k: stable order vs brute force
# ------------------------------------------------------------------------------------------------

def brute_topk(row, k):

    order = sorted(range(len(row)), key=lambda i: (-float(row[i]), i))

    return [float(row[i]) for i in order[:k]], order[:k]


@pytest.mark.parametrize("dtype", [torch.float32, BF16])
def test_topk_matches_brute_force_with_ties(dtype):

    g = torch.Generator().manual_seed(1)
    logits = torch.randint(-3, 4, (5, 300), generator=g).to(dtype)
    logits[0, 7] = float("-inf")
    values, indices = topk.topk(logits, 37)

    for r in range(5):

        bv, bi = brute_topk(logits[r].float().tolist(), 37)
        assert indices[r].tolist() == bi
        assert values[r].float().tolist() == bv


def test_topk_ties_go_to_lowest_index_not_topk_order():

    x = torch.zeros(1, 1000, dtype=BF16)
    values, indices = topk.topk(x, 128)
    assert indices[0].tolist() == list(range(128))


# ------------------------------------------------------------------------------------------------
# Prologue closed forms
# ------------------------------------------------------------------------------------------------

def tiny_state(vocab=64, **overrides):

    def bf(v):

        return torch.tensor([v], dtype=torch.float32).to(BF16)

    st = oracle.State(
        target=[0], draft=[0],
        grammar=torch.full((1, 1, (vocab + 31) // 32), -1, dtype=I32),
        context=torch.zeros(1, vocab, dtype=I32), decode=torch.zeros(1, vocab, dtype=I32),
        bias=torch.zeros(1, vocab, dtype=BF16),
        multiplicative=bf(1.0), frequency=bf(0.0), presence=bf(0.0), temperature=bf(1.0),
        top_p=bf(1.0), min_p=bf(0.0), top_k=torch.tensor([128], dtype=I32),
        top_logprobs=torch.tensor([0], dtype=I32),
        gumbel_target=torch.zeros(1, 1, vocab, dtype=BF16), gumbel_draft=torch.zeros(1, 1, vocab, dtype=BF16),
        uniform=torch.ones(1, 1, dtype=BF16),
    )

    for k, v in overrides.items():

        setattr(st, k, v)

    return st


def row(values, vocab=64):

    x = torch.full((vocab,), -1.0, dtype=BF16)
    x[: len(values)] = torch.tensor(values, dtype=torch.float32).to(BF16)

    return x


def test_multiplicative_penalty_closed_form():

    st = tiny_state(multiplicative=torch.tensor([2.0]).to(BF16))
    st.context[0, :2] = 1   # tokens 0 and 1 seen
    x = oracle.process_row(row([-2.0, 3.0, 3.0, -2.0]), st, 0, oracle.MULT, None, [], None)
    assert x[:4].float().tolist() == [-4.0, 1.5, 3.0, -2.0]


def test_frequency_presence_bias_temperature_closed_form():

    st = tiny_state(frequency=torch.tensor([0.5]).to(BF16), presence=torch.tensor([0.25]).to(BF16),
                    temperature=torch.tensor([2.0]).to(BF16))
    st.decode[0, 1] = 3
    st.bias[0, 2] = 1.5
    ind = oracle.FREQ | oracle.PRES | oracle.BIAS | oracle.TEMP
    x = oracle.process_row(row([1.0, 1.0, 1.0]), st, 0, ind, None, [], None)
    # token 1: (1 - 3 * 0.5 - 0.25) / 2 = -0.375 ; token 2: (1 + 1.5) / 2 = 1.25
    assert x[:3].float().tolist() == [0.5, -0.375, 1.25]


def test_frequency_penalty_rounds_once():
    """bf16(x - c * f) in one rounding (torch addcmul), not bf16(x - bf16(c * f))."""

    g = torch.Generator().manual_seed(0)
    found = None

    for _ in range(20000):

        x = float(torch.randn(1, generator=g).to(BF16) * 8)
        f = float((torch.rand(1, generator=g) * 2).to(BF16))
        c = int(torch.randint(1, 200, (1,), generator=g))
        single = float(torch.tensor(x - c * f, dtype=torch.float32).to(BF16))
        cf = float(torch.tensor(c * f, dtype=torch.float32).to(BF16))
        double = float(torch.tensor(x - cf, dtype=torch.float32).to(BF16))

        if single != double:

            found = (x, f, c, single)
            break

    assert found is not None
    x, f, c, single = found
    st = tiny_state(frequency=torch.tensor([f]).to(BF16))
    st.decode[0, 0] = c
    out = oracle.process_row(row([x]), st, 0, oracle.FREQ, None, [], None)
    assert float(out[0]) == single


def test_grammar_and_history():

    st = tiny_state(presence=torch.tensor([1.0]).to(BF16))
    st.grammar[0, 0, 0] = 0b1011   # tokens 0, 1, 3 allowed
    x = oracle.process_row(row([1.0, 1.0, 1.0, 1.0, 1.0]), st, 0, oracle.GRAMMAR | oracle.PRES,
                           st.grammar[0, 0], [0, 3, 0], None)
    # grammar masks 2 and 4; presence hits token 3 (history) but never token 0
    assert x[:5].float().tolist() == [1.0, 1.0, float("-inf"), 0.0, float("-inf")]


def test_d2t_reads_target_vocabulary_state():

    st = tiny_state(vocab=64, frequency=torch.tensor([1.0]).to(BF16))
    st.decode[0, 40] = 2
    d2t = torch.tensor([40, 3, 5, 7], dtype=torch.int64)
    x = oracle.process_row(row([1.0, 1.0, 1.0, 1.0], vocab=4), st, 0, oracle.FREQ, None, [], d2t)
    assert x.float().tolist() == [-1.0, 1.0, 1.0, 1.0]


# ------------------------------------------------------------------------------------------------
# Truncation by hand
# ------------------------------------------------------------------------------------------------

def logits_for(probs):

    p = torch.tensor(probs, dtype=torch.float64)

    return torch.log(p).to(torch.float32).to(BF16)[None]


def test_top_k_hand_case():

    st = tiny_state(top_k=torch.tensor([2], dtype=I32))
    v, _ = oracle.truncate(torch.tensor([[5.0, 4.0, 3.0, 2.0]]).to(BF16), oracle.TOP_K, st, 0)
    assert v[0].float().tolist() == [5.0, 4.0, float("-inf"), float("-inf")]


def test_top_p_masks_the_crossing_token():
    """mask = cumsum > p: with p = 0.6 and probabilities (0.5, 0.3, 0.2) only token 0 survives."""

    st = tiny_state(top_p=torch.tensor([0.6]).to(BF16))
    v, knife = oracle.truncate(logits_for([0.5, 0.3, 0.2]), oracle.TOP_P, st, 0)
    assert torch.isfinite(v[0]).tolist() == [True, False, False]
    assert not knife


def test_top_p_keeps_first_position_even_below():

    st = tiny_state(top_p=torch.tensor([0.1]).to(BF16))
    v, _ = oracle.truncate(logits_for([0.4, 0.35, 0.25]), oracle.TOP_P, st, 0)
    assert torch.isfinite(v[0]).tolist() == [True, False, False]


def test_min_p_hand_case():

    st = tiny_state(min_p=torch.tensor([0.2]).to(BF16))
    v, _ = oracle.truncate(logits_for([0.6, 0.3, 0.1]), oracle.MIN_P, st, 0)
    # lower = 0.2 * 0.6 = 0.12 > 0.1
    assert torch.isfinite(v[0]).tolist() == [True, True, False]


def test_min_p_compares_bf16_scores():
    """min-p compares bf16 scores with a bf16 threshold (reference core/naive.py:316-326: the
    softmax of bf16 values is bf16, and so is min_p times its first entry). Logits (0, -1.203125,
    -4) have probabilities 0.758397, 0.227712, 0.013891 and min_p = bf16(0.3) = 0.30078125. In
    bf16 the scores are 0.7578125 and 0.2275390625, and the threshold bf16(0.30078125 * 0.7578125
    = 0.227936) = 0.2275390625 equals the second score, which stays. With fp32 scores the second
    (0.227712) falls below 0.30078125 * 0.758397 = 0.228112 and would be masked. Every rounding
    above sits at least 0.1 bf16 ulp from a rounding boundary."""

    st = tiny_state(min_p=torch.tensor([0.3]).to(BF16))
    assert float(st.min_p[0]) == 0.30078125
    x = torch.tensor([[0.0, -1.203125, -4.0]]).to(BF16)
    v, knife = oracle.truncate(x.clone(), oracle.MIN_P, st, 0)
    assert torch.isfinite(v[0]).tolist() == [True, True, False]
    assert not knife
    # the fp32 formulation decides the other way on the same row
    s32 = x.float().softmax(-1)
    assert float(s32[0, 1]) < 0.30078125 * float(s32[0, 0])


# ------------------------------------------------------------------------------------------------
# Selection and verification invariants
# ------------------------------------------------------------------------------------------------

def stochastic_state(rows, vocab, seed):

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    b = SamplingBuffers.default(size=rows, timesteps=4, vocab_size=vocab, device="cpu")
    b.flags = Flags.from_values(rows, 4, Indicator.TOP_K_LOGPROBS, device="cpu")
    b.top_logprobs.fill_(5)

    return b, oracle.State.from_buffers(b)


def test_zero_noise_selects_the_maximum():

    b, st = stochastic_state(4, 512, 0)
    st.gumbel_target.zero_()
    logits = torch.randn(4, 512).to(BF16)
    res = oracle.singular(logits, st, scope="target")
    assert [r.token for r in res] == logits.float().argmax(-1).tolist()


def test_noise_can_force_any_candidate():

    b, st = stochastic_state(2, 512, 0)
    st.gumbel_target.fill_(0.0)
    logits = torch.randn(2, 512).to(BF16)
    # a very negative w on a non-maximal candidate that is inside the top-128
    target = int(logits[0].float().argsort(descending=True)[5])
    st.gumbel_target[0, 0, target] = -1000.0
    res = oracle.singular(logits, st, scope="target")
    assert res[0].token == target


def test_logprobs_are_log_softmax_of_the_support():

    b, st = stochastic_state(3, 1024, 1)
    logits = (torch.randn(3, 1024) * 3).to(BF16)
    res = oracle.singular(logits, st, scope="target", logprobs=True, max_top_logprobs=5)

    for r, rec in enumerate(res):

        v = logits[r].float().sort(descending=True).values[:128].double()
        lse = torch.logsumexp(v, 0)
        assert abs(rec.top_logprobs[0] - float(v[0] - lse)) < 1e-5
        assert rec.logprob <= 0


def verification_case(drafted, gamma=3, vocab=256, probs=None, uniform=None, seed=0):

    b, st = stochastic_state(1, vocab, seed)
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(gamma + 1, vocab, generator=g) * 2).to(BF16)

    if uniform is not None:

        st.uniform[0, :gamma + 1] = torch.tensor(uniform, dtype=torch.float32).to(BF16)

    res = oracle.multistep(logits, st, torch.tensor(drafted, dtype=I32), [0, gamma + 1],
                           probabilities=probs, logprobs=True)

    return res[0], logits, st


def test_point_mass_draft_of_argmax_is_accepted_with_u_below_p():

    gamma = 3
    _, logits, _ = verification_case([0] * (gamma + 1))
    drafted = logits.float().argmax(-1).tolist()
    rec, _, _ = verification_case(drafted, uniform=[1e-3] * (gamma + 1))
    assert rec.offset == gamma
    assert rec.tokens[:gamma] == drafted[:gamma]


def test_draft_outside_support_is_rejected():

    gamma = 3
    _, logits, _ = verification_case([0] * (gamma + 1))
    worst = logits[0].float().argmin().item()
    rec, _, _ = verification_case([worst, 1, 1, 1], uniform=[1e-3] * (gamma + 1))
    assert rec.offset == 0
    assert rec.tokens[0] != worst


def test_residual_picks_the_only_positive_candidate():
    """q = p on every candidate but one: the residual max(p - q, 0) leaves only that one."""

    gamma, vocab = 2, 256
    rec0, logits, st = verification_case([1, 2, 3], gamma=gamma, vocab=vocab, uniform=[1.0, 1.0, 1.0])
    v, idx = oracle.bounded(logits[0].float().to(BF16)[None])
    p = torch.log_softmax(v.float(), -1).exp()[0]
    q = torch.zeros(1, gamma, vocab)
    q[0, 0, idx[0].long()] = p
    keep = int(idx[0, 3])
    q[0, 0, keep] = 0.0
    drafted = [int(idx[0, 0]), 2, 3]
    q[0, 0, drafted[0]] = 1.0      # u q = 1 > p: the first draft is rejected
    rec, _, _ = verification_case(drafted, gamma=gamma, vocab=vocab, probs=q.to(BF16), uniform=[1.0, 1.0, 1.0])
    assert rec.offset == 0
    assert rec.tokens == [keep]


def test_offsets_and_emitted_prefix_invariants():

    g = torch.Generator().manual_seed(3)

    for seed in range(10):

        drafted = torch.randint(0, 256, (4,), generator=g).tolist()
        rec, _, _ = verification_case(drafted, seed=seed)
        assert 0 <= rec.offset <= 3
        assert rec.tokens[:rec.offset] == drafted[:rec.offset]
        assert len(rec.logprobs) == rec.offset + 1
        assert all(lp <= 0 for lp in rec.logprobs)


# ------------------------------------------------------------------------------------------------
# Cross-check against the batch-level restatement (sonic_sampler.core.NaiveSampler)
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("indicator", [0x3BE, 0x5BE, 0x41, 0x2A])
def test_per_row_oracle_matches_batch_naive(indicator):

    from sonic_sampler.core import NaiveSampler
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    rows, vocab = 6, 4096
    b = SamplingBuffers.random(size=rows, timesteps=2, vocab_size=vocab, device="cpu", seed=indicator,
                               indicators=Indicator(indicator), max_top_logprobs=5)
    logits = (torch.randn(rows, vocab, generator=torch.Generator().manual_seed(indicator)) * 3).to(BF16)

    naive = NaiveSampler(buffers=b, max_top_logprobs=5)
    expected = naive.singular(logits.clone(), None, 0, prefill=True, logprobs=True)
    st = oracle.State.from_buffers(b)
    res = oracle.singular(logits, st, scope="target", logprobs=True, max_top_logprobs=5)

    assert [r.token for r in res] == expected.tokens[:, 0].tolist()

    for r, rec in enumerate(res):

        assert float(torch.tensor(rec.logprob).to(BF16)) == float(expected.logprobs.selected[r, 0])


# ------------------------------------------------------------------------------------------------
# Decode-count updates, top-Z limits and the multistep history, by hand
# (reference ops/singular.py:134-151, ops/verify.py:75-91,425-429, ops/singular.py:335-346,
# core/naive.py:179-203)
# ------------------------------------------------------------------------------------------------

def slots_state(slots, vocab, indicator, timesteps=4):
    """A state of `slots` requests sharing one indicator word, every processor neutral."""

    def bf(v):

        return torch.full((slots,), v, dtype=torch.float32).to(BF16)

    return oracle.State(
        target=[indicator] * slots, draft=[indicator] * slots,
        grammar=torch.full((slots, timesteps, (vocab + 31) // 32), -1, dtype=I32),
        context=torch.zeros(slots, vocab, dtype=I32), decode=torch.zeros(slots, vocab, dtype=I32),
        bias=torch.zeros(slots, vocab, dtype=BF16),
        multiplicative=bf(1.0), frequency=bf(0.0), presence=bf(0.0), temperature=bf(1.0),
        top_p=bf(1.0), min_p=bf(0.0), top_k=torch.full((slots,), 128, dtype=I32),
        top_logprobs=torch.zeros(slots, dtype=I32),
        gumbel_target=torch.zeros(slots, timesteps, vocab, dtype=BF16),
        gumbel_draft=torch.zeros(slots, timesteps, vocab, dtype=BF16),
        uniform=torch.ones(slots, timesteps, dtype=BF16),
    )


def peaked(vocab, peaks):
    """bf16 rows of -4 with a unique maximum 8 at column peaks[r]."""

    x = torch.full((len(peaks), vocab), -4.0)

    for r, c in enumerate(peaks):

        x[r, c] = 8.0

    return x.to(BF16)


def test_singular_count_update_adds_one_at_the_slot():

    st = slots_state(4, 64, oracle.GREEDY)
    st.decode[2, 7] = 5
    st.decode[0, 7] = 9      # the same token in another slot must not move
    res = oracle.singular(peaked(64, [7, 11]), st, slot_mapping=[2, 3])
    assert [r.token for r in res] == [7, 11]
    after = oracle.apply_singular_counts(st.decode, res, [2, 3], prefill=False)
    assert int(after[2, 7]) == 6 and int(after[3, 11]) == 1 and int(after[0, 7]) == 9
    assert int((after != st.decode).sum()) == 2


def test_singular_prefill_stores_one():
    """Prefill writes 1 whatever the count held (reference ops/singular.py:143-145)."""

    st = slots_state(2, 64, oracle.GREEDY)
    st.decode[1, 7] = 5
    res = oracle.singular(peaked(64, [30, 7]), st)
    after = oracle.apply_singular_counts(st.decode, res, None, prefill=True)
    assert int(after[1, 7]) == 1 and int(after[0, 30]) == 1
    assert int((after != st.decode).sum()) == 2


def test_drafted_count_update_lands_at_the_target_id():
    """With d2t the update is at the remapped (target-vocabulary) id, in the row's slot."""

    st = slots_state(2, 64, oracle.GREEDY)
    d2t = torch.tensor([40, 3, 5, 7], dtype=torch.int64)
    res = oracle.singular(peaked(4, [0]), st, scope="draft", slot_mapping=[1], d2t=d2t)
    assert res[0].token == 40
    after = oracle.apply_singular_counts(st.decode, res, [1], prefill=False)
    assert int(after[1, 40]) == 1 and int(after[1, 0]) == 0 and int(after.sum()) == 1


def test_multistep_counts_add_one_per_emitted_token_including_the_bonus():

    vocab = 64
    st = slots_state(3, vocab, oracle.GREEDY)
    # request 0 (slot 2): argmax 9, 9, 12, 30 and drafts 9, 9, 5: two accepted, then 12
    # request 1 (slot 0): every draft equals the argmax: three accepted plus the bonus 33
    peaks = [9, 9, 12, 30, 20, 21, 22, 33]
    drafted = torch.tensor([9, 9, 5, 0, 20, 21, 22, 0], dtype=I32)
    st.decode[2, 9] = 1
    res = oracle.multistep(peaked(vocab, peaks), st, drafted, [0, 4, 8], slot_mapping=[2, 0])
    assert [r.offset for r in res] == [2, 3]
    assert res[0].tokens == [9, 9, 12] and res[1].tokens == [20, 21, 22, 33]
    after = oracle.apply_multistep_counts(st.decode, res, [2, 0])
    assert int(after[2, 9]) == 3 and int(after[2, 12]) == 1 and int(after[2, 5]) == 0
    assert [int(after[0, t]) for t in (20, 21, 22, 33)] == [1, 1, 1, 1]
    assert int(after.sum()) == int(st.decode.sum()) + 7


def test_top_logprobs_follow_the_row_limit_and_the_0x400_bit():

    vocab = 256
    st = slots_state(3, vocab, oracle.TOP_K_LOGPROBS)
    st.target[1] = 0                                   # 0x400 off: no top logprobs at all
    st.top_logprobs = torch.tensor([2, 9, 9], dtype=I32)   # slot 2: 9 > Z, capped at Z = 5
    logits = torch.randn(3, vocab, generator=torch.Generator().manual_seed(4)).mul(2).to(BF16)
    res = oracle.singular(logits, st, logprobs=True, max_top_logprobs=5)
    assert [len(r.top_tokens) for r in res] == [2, 0, 5]
    assert [len(r.top_logprobs) for r in res] == [2, 0, 5]
    order = logits[0].float().sort(descending=True, stable=True).indices
    assert res[0].top_tokens == order[:2].tolist()
    v = logits[0].float().sort(descending=True).values[:128].double()
    assert abs(res[0].top_logprobs[1] - float(v[1] - torch.logsumexp(v, 0))) < 1e-5


def test_multistep_top_logprobs_per_emitted_position():

    vocab, n = 256, 4
    st = slots_state(1, vocab, oracle.TOP_K_LOGPROBS)
    st.top_logprobs = torch.tensor([3], dtype=I32)
    logits = torch.randn(n, vocab, generator=torch.Generator().manual_seed(5)).mul(2).to(BF16)
    st.uniform.fill_(0.0)                              # u = 0: every point-mass draft is accepted
    drafted = logits.float().argmax(-1).to(I32)
    res = oracle.multistep(logits, st, drafted, [0, n], logprobs=True, max_top_logprobs=20)
    assert res[0].offset == n - 1
    assert [len(t) for t in res[0].top_tokens] == [3] * n
    st.target[0] = 0
    res = oracle.multistep(logits, st, drafted, [0, n], logprobs=True, max_top_logprobs=20)
    assert [len(t) for t in res[0].top_tokens] == [0] * n


def test_multistep_history_is_the_earlier_drafts():
    """Step i is penalized by drafts[:i] (presence 2): with drafts (5, 6), step 1 must see 5
    penalized (5 -> -1 < 6 = 0.5) and accept 6, and the bonus step sees both. Without the history
    step 1 rejects; counting step i's own draft rejects step 0."""

    vocab = 64
    st = slots_state(1, vocab, oracle.GREEDY | oracle.PRES)
    st.presence = torch.tensor([2.0]).to(BF16)
    x = torch.full((3, vocab), -4.0)
    x[:, 5], x[:, 6] = 1.0, 0.5
    res = oracle.multistep(x.to(BF16), st, torch.tensor([5, 6, 0], dtype=I32), [0, 3])
    assert res[0].offset == 2 and res[0].tokens == [5, 6, 5]


def test_multistep_history_never_counts_token_0():
    """Drafts of token 0 add nothing to the history (the reference pads with 0 and restores the
    count of token 0): step 1 keeps token 0 at 1.0 above token 6 at 0.5."""

    vocab = 64
    st = slots_state(1, vocab, oracle.GREEDY | oracle.PRES)
    st.presence = torch.tensor([2.0]).to(BF16)
    x = torch.full((3, vocab), -4.0)
    x[:, 0], x[:, 6] = 1.0, 0.5
    res = oracle.multistep(x.to(BF16), st, torch.tensor([0, 0, 0], dtype=I32), [0, 3])
    assert res[0].offset == 2 and res[0].tokens == [0, 0, 0]
    # a counted token 0 in the slot's own decode counts does apply
    st.decode[0, 0] = 1
    res = oracle.multistep(x.to(BF16), st, torch.tensor([6, 0, 0], dtype=I32), [0, 3])
    assert res[0].tokens[0] == 6


# ------------------------------------------------------------------------------------------------
# The batched restatement (bench.py's CPU baseline) against the per-row one
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("indicator", [None, 0x3BF, 0x5BE, 0x41, 0x7A0])
def test_batched_oracle_matches_per_row(indicator):

    from oracle import batch
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    rows, vocab = 12, 4096
    seed = 7 if indicator is None else indicator
    b = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                               indicators=None if indicator is None else Indicator(indicator),
                               max_top_logprobs=5)
    logits = (torch.randn(rows, vocab, generator=torch.Generator().manual_seed(seed)) * 3).to(BF16)
    st = oracle.State.from_buffers(b)

    got = batch.singular(logits, st, max_top_logprobs=5)
    res = oracle.singular(logits, st, scope="target", logprobs=True, max_top_logprobs=5)

    assert got.tokens.tolist() == [r.token for r in res]

    for r, rec in enumerate(res):

        assert float(got.logprobs[r]) == rec.logprob
        z = len(rec.top_tokens)
        assert got.top_tokens[r, :z].tolist() == rec.top_tokens
        assert got.top_logprobs[r, :z].tolist() == rec.top_logprobs
        assert bool((got.top_tokens[r, z:] == -1).all())


def test_batched_oracle_on_config1_rows():

    import bench
    from oracle import batch

    work = bench.c1_workload(batch=8, vocab=32768)
    st = oracle.State.from_buffers(work.buffers)
    got = batch.singular(work.logits, st, max_top_logprobs=5)
    res = oracle.singular(work.logits, st, scope="target", logprobs=True, max_top_logprobs=5)
    assert got.tokens.tolist() == [r.token for r in res]
    assert got.logprobs.tolist() == [r.logprob for r in res]


def test_batched_oracle_reference_topk_formulation():
    """The reference's own bounded path, ``logits.topk(k=128)`` (core/naive.py:336), which the CPU
    baseline times, selects the same 128 values per row as the stable sort; on rows whose
    selection involves no tied value it also picks the same tokens with the same logprobs."""

    import bench
    from oracle import batch

    work = bench.c1_workload(batch=8, vocab=32768)
    st = oracle.State.from_buffers(work.buffers)
    by_sort = batch.singular(work.logits, st, max_top_logprobs=5)
    by_topk = batch.singular(work.logits, st, max_top_logprobs=5, bounded="topk")
    assert by_topk.tokens.tolist() == by_sort.tokens.tolist()
    assert by_topk.logprobs.tolist() == by_sort.logprobs.tolist()
    with pytest.raises(ValueError):
        batch.singular(work.logits, st, bounded="heap")


def test_logprob_tolerance_floor():
    """The absolute floor admits the other bf16 rounding of a logprob near 0 whose fp32 value sits
    a few ulp of log(s) from a rounding boundary, and nothing further away."""

    e = -0.0017128810286521912          # fp32 log-softmax value near a bf16 midpoint
    assert not oracle.bf16_within(-0.001708984375, e)
    assert oracle.bf16_within(-0.001708984375, e, floor=oracle.LOGPROB_FLOOR)
    assert oracle.bf16_within(-0.0017166137695, e, floor=oracle.LOGPROB_FLOOR)
    assert not oracle.bf16_within(-0.0017013549805, e, floor=oracle.LOGPROB_FLOOR)
    # away from 0 the relative band governs
    assert oracle.bf16_within(-3.0, -3.0000001, floor=oracle.LOGPROB_FLOOR)
    assert not oracle.bf16_within(-3.015625, -3.0, floor=oracle.LOGPROB_FLOOR)


@pytest.mark.parametrize("seed", [3, 4])
def test_naive_drafting_with_d2t_matches_per_row(seed):

    from sonic_sampler.core import NaiveSampler
    from sonic_sampler.core.buffer import SamplingBuffers

    rows, gamma, t, vd, vt = 6, 3, 2, 1024, 4096
    g = torch.Generator().manual_seed(seed)
    b = SamplingBuffers.random(size=rows, timesteps=gamma + 1, vocab_size=vt, device="cpu", seed=seed,
                               max_top_logprobs=5)
    d2t = torch.randperm(vt, generator=g)[:vd]
    logits = (torch.randn(rows, vd, generator=g) * 3).to(BF16)
    tokens = torch.randint(1, vt, (rows, gamma + 1), generator=g).to(I32)

    got = NaiveSampler(buffers=b, max_top_logprobs=5).singular(logits, tokens, t, mapping=d2t, probs=True)
    st = oracle.State.from_buffers(b)
    res = oracle.singular(logits, st, scope="draft", timestep=t, d2t=d2t, drafted=tokens, history=t,
                          probs=True, max_top_logprobs=5)
    assert got.tokens[:, 0].tolist() == [r.token for r in res]

    for r, rec in enumerate(res):

        if rec.probs:

            for tok, v in rec.probs.items():

                assert float(got.probabilities[r, tok]) == float(torch.tensor(v).to(BF16))


@pytest.mark.parametrize("indicator", [None, 0x041, 0x4A0, 0x5BE])
def test_naive_multistep_matches_per_row(indicator):

    from sonic_sampler.core import NaiveSampler
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    batch, gamma, vocab = 5, 3, 2048
    n = gamma + 1
    seed = 9 if indicator is None else indicator
    g = torch.Generator().manual_seed(seed)
    b = SamplingBuffers.random(size=batch, timesteps=n, vocab_size=vocab, device="cpu", seed=seed,
                               indicators=None if indicator is None else Indicator(indicator),
                               max_top_logprobs=4)
    logits = (torch.randn(batch, n, vocab, generator=g) * 3).to(BF16)
    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch, n, generator=g) < 0.6, argmax,
                          torch.randint(1, vocab, (batch, n), generator=g)).to(I32)
    q = torch.softmax(torch.randn(batch, gamma, vocab, generator=g) * 2, dim=-1).to(BF16)

    ver, _ = NaiveSampler(buffers=b, max_top_logprobs=4).multistep(logits, drafted, q, logprobs=True)
    st = oracle.State.from_buffers(b)
    res = oracle.multistep(logits.view(batch * n, vocab), st, drafted.view(-1), list(range(0, batch * n + 1, n)),
                           probabilities=q, logprobs=True, max_top_logprobs=4)

    for r, rec in enumerate(res):

        if rec.knife:

            continue

        off = int(ver.offsets[r, 0])
        assert off == rec.offset, (r, off, rec.offset)
        assert ver.tokens[r, :off + 1].tolist() == rec.tokens

        for i, lp in enumerate(rec.logprobs):

            assert oracle.bf16_within(float(ver.logprobs.selected[r, i]), lp, floor=oracle.LOGPROB_FLOOR)
