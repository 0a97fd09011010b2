"""TEST INFRASTRUCTURE ONLY: CPU oracle for the WKV-7 recurrence.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the
timed CPU baseline). The product path in ``rwkv7m_amd`` never imports it.
"""

from .wkv_oracle import (  # noqa: F401
    backward,
    bf16_bits,
    bf16_from_bits,
    bf16_round,
    build,
    forward,
    normalized_max_error,
    np_backward,
    np_forward,
)
from . import screening_oracle, timemix_oracle  # noqa: F401,E402
