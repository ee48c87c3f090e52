"""Package logging (reference interface: fragpack/logging.py ``init_logger``).

Every module logger is a child of the ``fragpack_amd`` logger, which carries
the package's single stream handler and does not propagate, so a serving
engine's root handler never prints FragPack lines twice.  The level comes
from ``FRAGPACK_LOG_LEVEL`` (default INFO) when the package logger is first
configured; ``init_logger(..., level=...)`` sets one logger's own level.
"""

from __future__ import annotations

import logging
import os
import threading
from typing import IO

_ROOT = "fragpack_amd"
_FORMAT = "%(asctime)s %(levelname)s FragPack %(name)s %(message)s"
_setup = threading.Lock()
_handler: logging.Handler | None = None


def _package_logger(stream: IO[str] | None) -> logging.Logger:
    global _handler
    root = logging.getLogger(_ROOT)
    with _setup:
        if _handler is None or stream is not None:
            if _handler is not None:
                root.removeHandler(_handler)
            _handler = logging.StreamHandler(stream)
            _handler.setFormatter(logging.Formatter(_FORMAT))
            root.addHandler(_handler)
            root.setLevel(os.environ.get("FRAGPACK_LOG_LEVEL", "INFO").upper())
            root.propagate = False
    return root


def init_logger(name: str, level: str | None = None, stream: IO[str] | None = None) -> logging.Logger:
    """The logger for module ``name``, under the package logger.

    Args:
        name: Usually ``__name__``; names outside the package are placed under it.
        level: Optional level for this logger alone.
        stream: Optional stream for the package handler (replaces the previous one).
    """
    _package_logger(stream)
    full = name if name == _ROOT or name.startswith(_ROOT + ".") else f"{_ROOT}.{name}"
    logger = logging.getLogger(full)
    if level is not None:
        logger.setLevel(level.upper())
    return logger
