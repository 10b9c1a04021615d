from sonic_sampler.core.buffer import SamplingBuffers
from sonic_sampler.core.flags import SamplingMode, Indicator
from sonic_sampler.core.naive import NaiveSampler
