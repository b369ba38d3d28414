"""Stand-in for SGLang's forward context (``get_attn_backend``,
``get_token_to_kv_pool``): tests set ``ATTN_BACKEND`` and ``POOL``."""

ATTN_BACKEND = None
POOL = None


def get_attn_backend():
    return ATTN_BACKEND


def get_token_to_kv_pool():
    return POOL
