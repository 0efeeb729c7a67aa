"""Named loggers under the ``llmopt`` namespace.

Mirrors the logger helper the reference's quantization layer uses
(``src/llmopt/utils/logging.py:41-46``): ``get_logger("quant.nn")`` returns the
``llmopt.quant.nn`` logger, and ``LLMOPT_LOG_LEVEL`` sets the package level.
"""

from __future__ import annotations

import logging
import os

_ROOT = "llmopt"
_configured = False


def _configure_root() -> None:
    global _configured
    if _configured:
        return
    root = logging.getLogger(_ROOT)
    level = os.environ.get("LLMOPT_LOG_LEVEL", "WARNING").upper()
    root.setLevel(getattr(logging, level, logging.WARNING))
    if not root.handlers:
        handler = logging.StreamHandler()
        handler.setFormatter(logging.Formatter("%(asctime)s %(levelname)s %(name)s: %(message)s"))
        root.addHandler(handler)
    _configured = True


def get_logger(name: str) -> logging.Logger:
    """Return the ``llmopt.<name>`` logger, configuring the package root once."""
    _configure_root()
    return logging.getLogger(f"{_ROOT}.{name}" if name else _ROOT)
