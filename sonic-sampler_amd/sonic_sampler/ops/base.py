"""Constants shared by every kernel path (reference ``ops/base.py:24-31``)."""

from __future__ import annotations

# Upper bound on top-k and the width of every candidate block.
MAX_K: int = 128


def next_power_of_2(value: int) -> int:
    """Smallest power of two >= value; 0 and powers of two map to themselves."""

    return value if value.bit_count() <= 1 else 1 << value.bit_length()
