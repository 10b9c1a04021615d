"""The GPU Philox stream vs the numpy oracle (bit-exact words, bf16-rounded noise within an ulp)."""

import numpy as np
import pytest
import torch

from oracle.philox import gumbel_from_words, noise_words

pytestmark = pytest.mark.gpu


def test_raw_words_match_oracle():

    from sonic_sampler.noise import philox_words

    seed, offset = 0x1234_5678_9ABC_DEF0, 17
    print("philox raw words", flush=True)
    words = philox_words(seed, offset, 3, 2, 5000, device="cuda:0").cpu().numpy().view(np.uint32)
    assert np.array_equal(words, noise_words(seed, offset, 3, 2, 5000))


def test_gumbel_transform_matches_oracle():

    from sonic_sampler.noise import materialize_gumbel

    seed, offset = 99, 5
    noise = materialize_gumbel(seed, offset, 2, 3, 20000, device="cuda:0").float().cpu().numpy()
    expected = gumbel_from_words(noise_words(seed, offset, 2, 3, 20000))
    # log implementations may differ in the last fp32 bit, which moves a bf16 rounding rarely
    ulp = np.abs(expected) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(noise - expected) <= ulp)
    assert np.mean(noise == expected) > 0.999
    # log(Exp(1)) has mean -Euler-Mascheroni
    assert abs(float(noise.mean()) + 0.5772) < 0.02


@pytest.mark.parametrize("seed,offset,slots,steps,vocab", [
    (2 ** 64 - 1, 2 ** 32 - 1, 2, 2, 262144),       # every key and offset bit set, the widest vocabulary
    (0x0123_4567_89AB_CDEF, 0, 512, 65, 16),         # the last slot of 512 and timestep 64
])
def test_raw_words_at_the_counter_limits(seed, offset, slots, steps, vocab):

    from sonic_sampler.noise import philox_words

    print(f"philox words at the limits: slots={slots} steps={steps} vocab={vocab}", flush=True)
    words = philox_words(seed, offset, slots, steps, vocab, device="cuda:0").cpu().numpy().view(np.uint32)
    assert np.array_equal(words, noise_words(seed, offset, slots, steps, vocab))
