"""Package logger (reference: fragpack/logging.py:15-51).

``FRAGPACK_LOG_LEVEL`` selects the level (default INFO); one stream handler
per logger, propagation off so a serving engine's root handler does not
duplicate messages.
"""

from __future__ import annotations

import logging
import os
import threading
from typing import IO

_LOCK = threading.Lock()
_HANDLERS: dict[str, logging.Handler] = {}


def init_logger(name: str, level: str | None = None, stream: IO[str] | None = None) -> logging.Logger:
    with _LOCK:
        logger = logging.getLogger(name)
        handler = _HANDLERS.get(name)
        if handler is not None and stream is not None:
            logger.removeHandler(handler)
            handler.close()
            handler = None
        if handler is None:
            handler = logging.StreamHandler(stream)
            handler.setFormatter(logging.Formatter("%(asctime)s %(levelname)s FragPack %(name)s %(message)s"))
            logger.addHandler(handler)
            _HANDLERS[name] = handler
        logger.setLevel((level or os.environ.get("FRAGPACK_LOG_LEVEL", "INFO")).upper())
        logger.propagate = False
        return logger
