"""f32 values in the reference's JSON files (serde_json): decimal text read
with exact round-to-nearest-even to f32, and f32 written as the shortest
decimal that reads back to the same bits."""
from __future__ import annotations

from fractions import Fraction

import numpy as np

_INF = np.float32(np.inf)
_OVERFLOW = Fraction(float(np.finfo(np.float32).max)) + Fraction(2) ** 103


def f32_from_text(text: str) -> np.float32:
    """The f32 nearest the decimal number `text` (ties to even), as serde_json
    parses an f32 field: one rounding of the exact value, not decimal ->
    f64 -> f32."""
    t = text.strip()
    exact = Fraction(t)
    neg = t.startswith("-")
    if exact == 0:
        return np.float32(-0.0) if neg else np.float32(0.0)
    if abs(exact) >= _OVERFLOW:  # at or past max + half an ulp: rounds to infinity
        return np.float32(-np.inf) if neg else _INF
    with np.errstate(over="ignore"):
        x = np.float32(float(exact))  # within one f32 step of the answer
    best = None
    for c in (np.nextafter(x, -_INF), x, np.nextafter(x, _INF)):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - exact)
        if best is None or d < best[0] or (d == best[0] and int(c.view(np.uint32)) & 1 == 0):
            best = (d, c)
    return np.float32(best[1])


def f32_text(v) -> str:
    """Shortest decimal text that reads back as the same f32 (JSON number)."""
    v = np.float32(v)
    if not np.isfinite(v):
        raise ValueError("non-finite f32 has no JSON number form")
    a = abs(float(v))
    if a != 0.0 and (a < 1e-4 or a >= 1e16):
        return np.format_float_scientific(v, unique=True, trim="0")
    return np.format_float_positional(v, unique=True, trim="0")
