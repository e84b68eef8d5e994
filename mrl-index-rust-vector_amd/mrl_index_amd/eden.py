"""EdenFit (src/eden.rs:100-203): the corpus prefix mean shared by encode and query."""
from __future__ import annotations

import json
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .block import MRL_PREFIX_DIMS
from .jsonf32 import f32_from_text, f32_text

# eden.rs:15-44
LLOYD_MAX = {
    1: np.array([-0.79788456, 0.79788456], dtype=np.float32),
    4: np.array([-2.73258958, -2.06901724, -1.61804640, -1.25623121, -0.94234046, -0.65675912,
                 -0.38804830, -0.12839503, 0.12839503, 0.38804830, 0.65675912, 0.94234046,
                 1.25623121, 1.61804640, 2.06901724, 2.73258958], dtype=np.float32),
}


@dataclass
class EdenFit:
    dim: int
    bits: int
    seed: int
    mean: np.ndarray
    n_observed: int = 0

    def __post_init__(self):
        self.mean = np.ascontiguousarray(self.mean, dtype=np.float32)
        if self.mean.shape != (self.dim,):
            raise ValueError("mean must have dim entries")

    @classmethod
    def fit_band(cls, rows: np.ndarray, start: int, dim: int, bits: int, seed: int) -> "EdenFit":
        """eden.rs:130-159 (sequential f32 sum over rows, then *= 1/n)."""
        if not 1 <= bits <= 4 or dim & (dim - 1):
            raise ValueError("bits in 1..=4 and dim a power of two")
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        if rows.ndim != 2 or rows.shape[0] == 0:
            raise ValueError("empty corpus for EdenFit")
        mean = np.zeros(dim, dtype=np.float32)
        _lib.check(_lib.lib.mrl_eden_fit_band(_lib.fptr(rows), rows.shape[0], rows.shape[1], start, dim,
                                              _lib.fptr(mean)))
        return cls(dim, bits, seed, mean, rows.shape[0])

    @classmethod
    def fit_slice(cls, rows, dim, bits, seed):
        return cls.fit_band(rows, 0, dim, bits, seed)

    @classmethod
    def fit_prefix(cls, rows, bits=4, seed=1):
        return cls.fit_band(rows, 0, MRL_PREFIX_DIMS, bits, seed)

    @classmethod
    def zeros(cls, dim: int, bits: int, seed: int) -> "EdenFit":
        return cls(dim, bits, seed, np.zeros(dim, dtype=np.float32), 0)

    @classmethod
    def default_prefix(cls, seed: int = 1) -> "EdenFit":
        return cls.zeros(MRL_PREFIX_DIMS, 4, seed)

    def observe_prefix(self, x) -> None:
        """eden.rs:182-191: m <- m + (x - m) * (1/n), elementwise f32."""
        x = np.asarray(x, dtype=np.float32)[: self.dim]
        n = self.n_observed + 1
        inv = np.float32(1.0) / np.float32(n)
        self.mean = (self.mean + (x - self.mean) * inv).astype(np.float32)
        self.n_observed = n

    def to_c(self) -> _lib.EdenFitC:
        return _lib.EdenFitC(self.dim, self.bits, self.seed, _lib.fptr(self.mean), self.n_observed)

    def save_json(self, path) -> None:
        """eden.rs:193-197 (serde_json pretty form; f32 as shortest round-trip text)."""
        with open(path, "w") as f:
            f.write(self.to_json())

    def to_json(self) -> str:
        mean = ",\n".join("    " + f32_text(v) for v in self.mean)
        return (f'{{\n  "dim": {int(self.dim)},\n  "bits": {int(self.bits)},\n  "seed": {int(self.seed)},\n'
                f'  "mean": [\n{mean}\n  ],\n  "n_observed": {int(self.n_observed)}\n}}')

    @classmethod
    def load_json(cls, path) -> "EdenFit":
        """eden.rs:199-202.  Each mean value is rounded once from its decimal
        text to f32, as serde_json does; a missing n_observed is 0
        (#[serde(default)]).  Malformed files raise ValueError."""
        with open(path) as f:
            return cls.from_json(f.read())

    @classmethod
    def from_json(cls, text: str) -> "EdenFit":
        d = json.loads(text, parse_float=str)
        try:
            dim, bits, seed = _uint(d["dim"]), _uint(d["bits"], 255), _uint(d["seed"])
            mean = np.array([f32_from_text(_num(v)) for v in d["mean"]], dtype=np.float32)
            n_obs = _uint(d.get("n_observed", 0))
        except (KeyError, TypeError) as e:
            raise ValueError(f"eden fit json: {e!r}") from None
        return cls(dim, bits, seed, mean, n_obs)


def _uint(v, hi=2 ** 64 - 1) -> int:
    if isinstance(v, bool) or not isinstance(v, int) or not 0 <= v <= hi:
        raise ValueError(f"expected an unsigned integer, got {v!r}")
    return v


def _num(v) -> str:
    # parse_float=str hands decimals over as text; integers arrive as int
    if isinstance(v, bool) or not isinstance(v, (int, str)):
        raise ValueError(f"expected a number, got {v!r}")
    return str(v)
