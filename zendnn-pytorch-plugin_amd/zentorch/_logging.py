"""Package logger; level from ZENTORCH_PY_LOG_LEVEL, as in the reference
(src/cpu/python/zentorch/_logging.py:10-25)."""
import logging
import os


def get_logger(name):
    logger = logging.getLogger(name)
    level = os.environ.get("ZENTORCH_PY_LOG_LEVEL", "WARNING").upper()
    logger.setLevel(getattr(logging, level, logging.WARNING))
    if not logger.handlers:
        h = logging.StreamHandler()
        h.setFormatter(logging.Formatter("[%(name)s %(levelname)s] %(message)s"))
        logger.addHandler(h)
    return logger
