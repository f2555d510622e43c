"""``init_logger`` with vLLM's ``info_once`` (vllm/logger.py)."""
import logging


class _Logger(logging.LoggerAdapter):
    _seen: set = set()

    def info_once(self, msg, *args):
        key = (msg,) + tuple(args)
        if key not in self._seen:
            self._seen.add(key)
            self.info(msg, *args)


def init_logger(name):
    return _Logger(logging.getLogger(name), {})
