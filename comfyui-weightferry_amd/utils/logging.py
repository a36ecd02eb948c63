"""log_info / log_warn through the "WeightFerry" logger with the "[WeightFerry]" prefix (the reference's
utils/logging.py:21-36)."""
import logging

_logger = logging.getLogger("WeightFerry")


def log_info(msg):
    _logger.info("[WeightFerry] %s", msg)


def log_warn(msg):
    _logger.warning("[WeightFerry] %s", msg)
