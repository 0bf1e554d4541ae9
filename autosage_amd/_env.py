"""Environment lookups on the per-call path.

The operators and the scheduler read their switches from the environment on
every call, as the reference does (a change takes effect on the next call).
``os.getenv`` encodes the name and decodes the value on every lookup, about
1 µs each; a cached scheduler call reads about twenty of them, more than the
kernel of a small graph takes.  ``get`` reads CPython's own mapping behind
``os.environ`` (the encoded strings, kept in step with every assignment
through ``os.environ``) and decodes a value only the first time it is seen;
elsewhere it is ``os.environ.get``.
"""

from __future__ import annotations

import os
from typing import Optional

_KEYS: dict[str, bytes] = {}
_VALUES: dict[bytes, str] = {}
_MAX_VALUES = 4096


def get(name: str, default: Optional[str] = None) -> Optional[str]:
    """``os.environ.get(name, default)``."""
    env = os.environ
    data = getattr(env, "_data", None)
    encode = getattr(env, "encodekey", None)
    decode = getattr(env, "decodevalue", None)
    if not isinstance(data, dict) or encode is None or decode is None:
        return env.get(name, default)
    key = _KEYS.get(name)
    if key is None:
        key = encode(name)
        _KEYS[name] = key
    raw = data.get(key)
    if raw is None:
        return default
    value = _VALUES.get(raw)
    if value is None:
        value = decode(raw)
        if len(_VALUES) < _MAX_VALUES:
            _VALUES[raw] = value
    return value


def raw(names: tuple[str, ...]) -> tuple:
    """The current values of ``names`` (None when unset), cheap enough to key
    a memo of what is parsed from them."""
    return tuple(get(n) for n in names)
