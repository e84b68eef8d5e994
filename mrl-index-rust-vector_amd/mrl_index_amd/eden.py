"""EdenFit (src/eden.rs:382-485): the corpus prefix mean shared by encode and query."""
from __future__ import annotations

import json
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .block import MRL_PREFIX_DIMS

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
        with open(path, "w") as f:
            json.dump({"dim": self.dim, "bits": self.bits, "seed": self.seed,
                       "mean": [float(v) for v in self.mean], "n_observed": self.n_observed}, f, indent=2)

    @classmethod
    def load_json(cls, path) -> "EdenFit":
        with open(path) as f:
            d = json.load(f)
        return cls(d["dim"], d["bits"], d["seed"], np.array(d["mean"], dtype=np.float32), d.get("n_observed", 0))
