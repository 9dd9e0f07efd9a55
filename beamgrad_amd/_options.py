# SPDX-License-Identifier: MIT
"""Search options: ``BeamOptions`` with the reference's field names, defaults,
accepted values and error messages (reference
python/beamgrad/_options.py:53-172).

Every field has one normalizer here. It returns the value to store (a plain
``int``, ``float``, ``bool`` or tuple of ``int``) or raises the field's
``ValueError``; ``__post_init__`` applies them in field order, so the first
bad field reported is the same one the reference reports.
"""

from __future__ import annotations

import math
import numbers
from collections.abc import Iterable
from dataclasses import dataclass

# Largest beam the HIP engine runs (DBS_CUDA_MAX_BEAM in include/dbs_cuda.h).
CUDA_MAX_BEAM = 1024
# Integer options travel to the engine as 32-bit ints; larger ones are
# rejected, never wrapped.
INT32_MAX = 2**31 - 1


def _is_int(value) -> bool:
    """An integral number that is not a bool (NumPy integer scalars count)."""
    return isinstance(value, numbers.Integral) and not isinstance(value, bool)


def _int_within(value, lo: int, hi: int) -> int | None:
    return int(value) if _is_int(value) and lo <= value <= hi else None


def _finite_real(value) -> float | None:
    """``float(value)`` for a finite real that is not a bool, else None (ints
    past the float range included)."""
    if isinstance(value, bool) or not isinstance(value, numbers.Real):
        return None
    try:
        as_float = float(value)
    except OverflowError:
        return None
    return as_float if math.isfinite(as_float) else None


def _sequence(value) -> tuple | None:
    """A sequence given as a list, tuple, array or tensor, as a tuple; None
    for a string, bytes or anything not iterable."""
    items = value.tolist() if hasattr(value, "tolist") else value
    if isinstance(items, (str, bytes)) or not isinstance(items, Iterable):
        return None
    return tuple(items)


def _all_token_ids(items: tuple) -> bool:
    return all(_int_within(t, 0, INT32_MAX) is not None for t in items)


def _beam_size(value) -> int:
    n = _int_within(value, 1, INT32_MAX)
    if n is None:
        raise ValueError(f"beam_size must be a positive int (at most 2**31 - 1), got {value!r}")
    return n


def _eos_token(value) -> int | tuple[int, ...]:
    """-1, one token id, or two or more distinct ids in the order given (a
    sequence naming one distinct id collapses to that id)."""
    if _is_int(value):
        n = _int_within(value, -1, INT32_MAX)
        if n is None:
            raise ValueError(f"eos_token must be -1 (disabled) or a token id, got {value!r}")
        return n
    items = _sequence(value)
    if items is None:
        raise ValueError(f"eos_token must be -1 (disabled), a token id or a sequence of token ids, got {value!r}")
    if not items or not _all_token_ids(items):
        raise ValueError(f"eos_token must be a non-empty sequence of token ids, got {value!r}")
    seen: list[int] = []
    for t in items:
        if int(t) not in seen:
            seen.append(int(t))
    return seen[0] if len(seen) == 1 else tuple(seen)


def _min_length(value) -> int:
    n = _int_within(value, 0, INT32_MAX)
    if n is None:
        raise ValueError(f"min_length must be a non-negative int (at most 2**31 - 1), got {value!r}")
    return n


def _alpha(value) -> float:
    a = _finite_real(value)
    if a is None or a < 0.0:
        raise ValueError(f"length_penalty_alpha must be a finite, non-negative number, got {value!r}")
    return a


def _validate(value) -> bool:
    if not isinstance(value, bool):
        raise ValueError(f"validate_inputs must be a bool, got {value!r}")
    return value


def _banned(value) -> tuple[int, ...] | None:
    """None, or the banned ids as a tuple (an empty one becomes None)."""
    if value is None:
        return None
    items = _sequence(value)
    if items is None:
        raise ValueError(f"banned_tokens must be a sequence of token ids, got {value!r}")
    if not _all_token_ids(items):
        raise ValueError(f"banned_tokens must hold non-negative int token ids, got {items!r}")
    return tuple(int(t) for t in items) or None


def _ngram(value) -> int:
    n = _int_within(value, 0, INT32_MAX)
    if n is None:
        raise ValueError(f"no_repeat_ngram_size must be a non-negative int (at most 2**31 - 1), got {value!r}")
    return n


def _penalty(value) -> float:
    r = _finite_real(value)
    if r is None or r <= 0.0:
        raise ValueError(f"repetition_penalty must be a finite, positive number, got {value!r}")
    return r


_NORMALIZERS = (
    ("beam_size", _beam_size),
    ("eos_token", _eos_token),
    ("min_length", _min_length),
    ("length_penalty_alpha", _alpha),
    ("validate_inputs", _validate),
    ("banned_tokens", _banned),
    ("no_repeat_ngram_size", _ngram),
    ("repetition_penalty", _penalty),
)


@dataclass(frozen=True)
class BeamOptions:
    """Beam search configuration (same meaning as ``beamgrad.BeamOptions``).

    beam_size: beams ``K`` (the beam dimension of the input).
    eos_token: end-of-sequence id, ``-1`` to disable, or several ids (each
        finishes a beam, which is then carried forward with the one it emitted).
    min_length: EOS is masked until a hypothesis has this many tokens.
    length_penalty_alpha: GNMT exponent; beams rank by raw / ((5 + len) / 6)^alpha.
    validate_inputs: raise ValueError when a row the search reads holds NaN or +inf.
    banned_tokens: ids never selected.
    no_repeat_ngram_size: n > 0 blocks tokens repeating an n-gram of the beam's prefix.
    repetition_penalty: > 1 subtracts its log from tokens already in the prefix.
    """

    beam_size: int
    eos_token: int | tuple[int, ...] = -1
    min_length: int = 0
    length_penalty_alpha: float = 0.0
    validate_inputs: bool = True
    banned_tokens: tuple[int, ...] | None = None
    no_repeat_ngram_size: int = 0
    repetition_penalty: float = 1.0

    def __post_init__(self) -> None:
        normalized = {name: norm(getattr(self, name)) for name, norm in _NORMALIZERS}
        for name, value in normalized.items():
            object.__setattr__(self, name, value)

    @property
    def eos_tokens(self) -> tuple[int, ...]:
        """Every EOS id in the order given; () when EOS handling is off."""
        eos = self.eos_token
        if isinstance(eos, tuple):
            return eos
        return (eos,) if eos >= 0 else ()

    def eos_ids(self, vocab_size: int) -> tuple[int, ...]:
        """``eos_tokens``, each checked to lie below ``vocab_size``."""
        for t in self.eos_tokens:
            if t >= vocab_size:
                raise ValueError(f"eos_token {t} is outside the vocabulary (size {vocab_size})")
        return self.eos_tokens

    def native_eos(self) -> tuple[int, list[int]]:
        """(eos_token, extra_eos) as the operators take them: the first id (-1
        when off) and the rest."""
        first, *rest = self.eos_tokens or (-1,)
        return first, list(rest)

    def banned_ids(self, vocab_size: int) -> tuple[int, ...] | None:
        """The banned ids, checked to lie below ``vocab_size``; None if none."""
        ids = self.banned_tokens
        if ids and any(t >= vocab_size for t in ids):
            raise ValueError(f"banned_tokens {ids} include ids outside the vocabulary (size {vocab_size})")
        return ids or None

    def banned_mask(self, vocab_size: int) -> list[int] | None:
        """The banned ids as a 0/1 list of ``vocab_size`` entries; None if none."""
        ids = self.banned_ids(vocab_size)
        if ids is None:
            return None
        marks = bytearray(vocab_size)
        for t in ids:
            marks[t] = 1
        return list(marks)
