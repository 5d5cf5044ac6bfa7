"""Utilities (logging) shared with the reference's API."""

from mlx_primitives.utils.logging import get_logger, log_fallback

__all__ = ["get_logger", "log_fallback"]
