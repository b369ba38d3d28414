"""Stand-in for SGLang's runtime context (``get_parallel``, ``process_model_config``):
tests set ``PARALLEL`` and ``MODEL_CONFIG``."""

from types import SimpleNamespace

PARALLEL = SimpleNamespace(tp_size=4, tp_rank=0, tp_group=None)
MODEL_CONFIG = SimpleNamespace(context_len=32768)


def get_parallel():
    return PARALLEL


def process_model_config():
    return MODEL_CONFIG
