from sonic_sampler.ops.base import MAX_K, next_power_of_2
