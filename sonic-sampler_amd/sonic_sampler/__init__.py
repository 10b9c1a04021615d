"""MI355X-native SonicSampler: fused sampling and speculative verification on gfx950.

The public surface mirrors the reference package ``sonic_sampler`` (``base``, ``core``,
``interface``, ``ops``); every sampling call runs hand-written HIP kernels through the C-ABI in
``include/sonic_sampler.h``.
"""

__version__ = "1.0.0"
