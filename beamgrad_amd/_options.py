# SPDX-License-Identifier: MIT
"""Search options, with the reference's fields, defaults and validation
(reference python/beamgrad/_options.py:53-172)."""

from __future__ import annotations

import math
import numbers
from collections.abc import Iterable
from dataclasses import dataclass

# Largest beam the HIP engine runs (DBS_CUDA_MAX_BEAM in include/dbs_cuda.h).
CUDA_MAX_BEAM = 1024
INT32_MAX = 2**31 - 1


def _is_int(value) -> bool:
    # bool is an int subclass, but not a count
    return isinstance(value, numbers.Integral) and not isinstance(value, bool)


def _finite(value) -> float | None:
    if not isinstance(value, numbers.Real) or isinstance(value, bool):
        return None
    try:
        out = float(value)
    except OverflowError:
        return None
    return out if math.isfinite(out) else None


def _token_list(value, what: str):
    if hasattr(value, "tolist"):
        value = value.tolist()
    if isinstance(value, (str, bytes)) or not isinstance(value, Iterable):
        raise ValueError(f"{what} must be a sequence of token ids, got {value!r}")
    return tuple(value)


def _normalize_eos(value) -> int | tuple[int, ...]:
    if _is_int(value):
        if not -1 <= value <= INT32_MAX:
            raise ValueError(f"eos_token must be -1 (disabled) or a token id, got {value!r}")
        return int(value)
    if hasattr(value, "tolist"):
        value = value.tolist()
    if isinstance(value, (str, bytes)) or not isinstance(value, Iterable):
        raise ValueError(f"eos_token must be -1 (disabled), a token id or a sequence of token ids, got {value!r}")
    tokens = tuple(value)
    if not tokens or any(not _is_int(t) or not 0 <= t <= INT32_MAX for t in tokens):
        raise ValueError(f"eos_token must be a non-empty sequence of token ids, got {value!r}")
    distinct = tuple(dict.fromkeys(int(t) for t in tokens))
    return distinct[0] if len(distinct) == 1 else distinct


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
        if not _is_int(self.beam_size) or not 1 <= self.beam_size <= INT32_MAX:
            raise ValueError(f"beam_size must be a positive int (at most 2**31 - 1), got {self.beam_size!r}")
        object.__setattr__(self, "eos_token", _normalize_eos(self.eos_token))
        if not _is_int(self.min_length) or not 0 <= self.min_length <= INT32_MAX:
            raise ValueError(f"min_length must be a non-negative int (at most 2**31 - 1), got {self.min_length!r}")
        alpha = _finite(self.length_penalty_alpha)
        if alpha is None or alpha < 0.0:
            raise ValueError(
                f"length_penalty_alpha must be a finite, non-negative number, got {self.length_penalty_alpha!r}")
        if not isinstance(self.validate_inputs, bool):
            raise ValueError(f"validate_inputs must be a bool, got {self.validate_inputs!r}")
        if self.banned_tokens is not None:
            banned = _token_list(self.banned_tokens, "banned_tokens")
            if any(not _is_int(t) or not 0 <= t <= INT32_MAX for t in banned):
                raise ValueError(f"banned_tokens must hold non-negative int token ids, got {banned!r}")
            object.__setattr__(self, "banned_tokens", tuple(int(t) for t in banned) or None)
        if not _is_int(self.no_repeat_ngram_size) or not 0 <= self.no_repeat_ngram_size <= INT32_MAX:
            raise ValueError(
                f"no_repeat_ngram_size must be a non-negative int (at most 2**31 - 1), got {self.no_repeat_ngram_size!r}")
        penalty = _finite(self.repetition_penalty)
        if penalty is None or penalty <= 0.0:
            raise ValueError(f"repetition_penalty must be a finite, positive number, got {self.repetition_penalty!r}")
        for name in ("beam_size", "min_length", "no_repeat_ngram_size"):
            object.__setattr__(self, name, int(getattr(self, name)))
        object.__setattr__(self, "length_penalty_alpha", alpha)
        object.__setattr__(self, "repetition_penalty", penalty)

    @property
    def eos_tokens(self) -> tuple[int, ...]:
        if isinstance(self.eos_token, tuple):
            return self.eos_token
        return () if self.eos_token < 0 else (self.eos_token,)

    def eos_ids(self, vocab_size: int) -> tuple[int, ...]:
        outside = [t for t in self.eos_tokens if t >= vocab_size]
        if outside:
            raise ValueError(f"eos_token {outside[0]} is outside the vocabulary (size {vocab_size})")
        return self.eos_tokens

    def native_eos(self) -> tuple[int, list[int]]:
        """(eos_token, extra_eos) as the operators take them."""
        tokens = self.eos_tokens
        return (tokens[0], list(tokens[1:])) if tokens else (-1, [])

    def banned_ids(self, vocab_size: int) -> tuple[int, ...] | None:
        if not self.banned_tokens:
            return None
        if max(self.banned_tokens) >= vocab_size:
            raise ValueError(
                f"banned_tokens {self.banned_tokens} include ids outside the vocabulary (size {vocab_size})")
        return self.banned_tokens

    def banned_mask(self, vocab_size: int) -> list[int] | None:
        ids = self.banned_ids(vocab_size)
        if ids is None:
            return None
        mask = [0] * vocab_size
        for token in ids:
            mask[token] = 1
        return mask
