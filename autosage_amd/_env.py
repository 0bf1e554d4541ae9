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
_NAME_KEYS: dict[tuple, tuple] = {}
_VALUES: dict[bytes, str] = {}
_MAX_VALUES = 4096
# (os.environ object, its encoded mapping or None, encodekey, decodevalue)
_STATE: Optional[tuple] = None


def _state() -> tuple:
    global _STATE
    env = os.environ
    state = _STATE
    if state is None or state[0] is not env:
        data = getattr(env, "_data", None)
        encode = getattr(env, "encodekey", None)
        decode = getattr(env, "decodevalue", None)
        usable = isinstance(data, dict) and encode is not None and decode is not None
        state = (env, data if usable else None, encode, decode)
        _STATE = state
    return state


def _key(name: str, encode) -> bytes:
    key = _KEYS.get(name)
    if key is None:
        key = encode(name)
        _KEYS[name] = key
    return key


def get(name: str, default: Optional[str] = None) -> Optional[str]:
    """``os.environ.get(name, default)``."""
    env, data, encode, decode = _state()
    if data is None:
        return env.get(name, default)
    raw_value = data.get(_key(name, encode))
    if raw_value is None:
        return default
    value = _VALUES.get(raw_value)
    if value is None:
        value = decode(raw_value)
        if len(_VALUES) < _MAX_VALUES:
            _VALUES[raw_value] = value
    return value


def raw(names: tuple[str, ...]) -> tuple:
    """The current values of ``names`` (None when unset), undecoded where the
    platform allows: a cheap key for a memo of what is parsed from them."""
    env, data, encode, _ = _state()
    if data is None:
        return tuple(env.get(n) for n in names)
    keys = _NAME_KEYS.get(names)
    if keys is None:
        keys = tuple(_key(n, encode) for n in names)
        _NAME_KEYS[names] = keys
    return tuple(map(data.get, keys))
