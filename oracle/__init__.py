"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

NumPy restatements of the reference algorithms (each function cites the
mlx-primitives file:line it follows). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package, and only as the
checker or the timed CPU baseline; the product path never does.

Parity pins are listed in tests/test_oracle.py; no oracle function is left
unpinned.
"""

from oracle import attention, attention_grad, kv_cache, paged  # noqa: F401
