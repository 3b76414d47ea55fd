"""Environment helpers (reference ``nanochat/train_utils.py:6-13``)."""

import os


def env_int(name: str, default_value: int) -> int:
    v = os.getenv(name)
    if v is None:
        return default_value
    try:
        return int(v)
    except ValueError:
        raise ValueError(f"{name} must be an integer, got: {v}")
