"""Small shared helpers (logging)."""

from llmopt.utils.logging import get_logger

__all__ = ["get_logger"]
