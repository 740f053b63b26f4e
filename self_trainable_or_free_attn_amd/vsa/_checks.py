"""Argument checks shared by the VSA configuration dataclasses. The messages are the reference's (they are part
of the interface callers may match on): "<Class>.<field> must be a real number / finite and >= 0 / an int /
>= 1"."""
import math


def _is_number(v, integral):
    if isinstance(v, bool):
        return False
    return isinstance(v, int) if integral else isinstance(v, (int, float))


def nonnegative_reals(obj, *fields):
    """Every named field of obj is a finite real number >= 0 (bool refused)."""
    owner = type(obj).__name__
    for f in fields:
        v = getattr(obj, f)
        if not _is_number(v, integral=False):
            raise TypeError(f"{owner}.{f} must be a real number, got {type(v).__name__}")
        if not (math.isfinite(v) and v >= 0):
            raise ValueError(f"{owner}.{f} must be finite and >= 0, got {v!r}")


def positive_ints(obj, *fields, optional=()):
    """Every named field of obj is an int >= 1 (bool refused); fields listed in `optional` may also be None."""
    owner = type(obj).__name__
    for f in fields:
        v = getattr(obj, f)
        if v is None and f in optional:
            continue
        if not _is_number(v, integral=True):
            raise TypeError(f"{owner}.{f} must be an int, got {type(v).__name__}")
        if v < 1:
            raise ValueError(f"{owner}.{f} must be >= 1, got {v!r}")
