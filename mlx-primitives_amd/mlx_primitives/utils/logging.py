"""The ``mlx_primitives`` logger (same name and env var as the reference's
mlx_primitives/utils/logging.py:30-108).

The MI355X build has no fallback path, so ``log_fallback`` is only kept for
callers that use it; kernel failures raise.
"""

from __future__ import annotations

import logging
import os
import threading
from typing import Optional

_logger: Optional[logging.Logger] = None
_lock = threading.Lock()
_seen: set = set()
_LEVELS = {"DEBUG", "INFO", "WARNING", "ERROR", "CRITICAL"}


def get_logger() -> logging.Logger:
    """Logger "mlx_primitives", level from MLX_PRIMITIVES_LOG_LEVEL (default WARNING)."""
    global _logger
    if _logger is None:
        with _lock:
            if _logger is None:
                lg = logging.getLogger("mlx_primitives")
                level = os.environ.get("MLX_PRIMITIVES_LOG_LEVEL", "WARNING").upper()
                lg.setLevel(getattr(logging, level if level in _LEVELS else "WARNING"))
                if not lg.handlers:
                    h = logging.StreamHandler()
                    h.setFormatter(logging.Formatter("%(name)s - %(levelname)s - %(message)s"))
                    lg.addHandler(h)
                _logger = lg
    return _logger


def log_fallback(operation: str, exception: Exception, context: Optional[str] = None) -> None:
    """Log a kernel failure: WARNING the first time per operation, DEBUG after."""
    with _lock:
        first = operation not in _seen
        _seen.add(operation)
    msg = f"{operation}: optimized kernel failed ({type(exception).__name__}: {exception})"
    if first:
        msg += " (first occurrence, further fallbacks logged at DEBUG)"
    if context:
        msg += f" | context: {context}"
    get_logger().log(logging.WARNING if first else logging.DEBUG, msg)
