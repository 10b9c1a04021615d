from sonic_sampler.base.buffer import Layout, SliceBuffer
from sonic_sampler.base.sampler import (
    LogProbabilities,
    Selection,
    TopTargets,
    Verification,
    DEFAULT_TOP_LOGPROBS,
)
from sonic_sampler.base.tensor import PrefixContiguousTensor, TimeDifferentiatedTensor
