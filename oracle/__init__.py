"""CPU oracle for the 4-bit group-quantized matmul path (test infrastructure only).

This package is a numpy restatement of the reference's algorithm. It is the
checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import it. The shipped path is the HIP
library under ``raceline_amd/``, which fails loudly when it is not built.
"""

from .q4 import *  # noqa: F401,F403
from .moe import *  # noqa: F401,F403
