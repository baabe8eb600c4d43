"""Seeded synthetic datasets for the benchmark configurations.

All draws use numpy's PCG64 with fixed seeds (stable for a given numpy
version), seeded as 0xF1A50000 + 16*config + stream with streams
0 = means, 1 = base, 2 = queries, 3 = signs.

  C1  N x 128 integer Gaussian mixture, 64 components: means ~ U[0,100]^d,
      x = max(0, rint(mu + 10 z)); queries from the same mixture.
  C2  as C1 with 1024 components (the headline configuration, N = 1M).
  C3  N x 96 unit vectors: 1024 components, means ~ N(0,1), x = mu + 0.3 z,
      normalised; queries = base point + N(0, 0.05), renormalised.
  C4  N x 960 in [0,1]: 256 components, means ~ U[0,1], x = clip(mu+0.1 z).
  C5  N x 1536 unit vectors: 4096 anisotropic components, means ~ N(0,1),
      per-component per-dimension scales s = 0.05 + 0.45 u (u ~ U[0,1]),
      x = mu + s * z, normalised; queries from the same mixture.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0xF1A50000


def _rng(config: int, stream: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED_BASE + 16 * config + stream))


def integer_mixture(n: int, nq: int, dim: int = 128, components: int = 64, config: int = 1,
                    sigma: float = 10.0):
    """C1/C2 generator: returns (base, queries) as float32 with integer values."""
    means = _rng(config, 0).uniform(0.0, 100.0, size=(components, dim)).astype(np.float32)

    def draw(count: int, stream: int) -> np.ndarray:
        r = _rng(config, stream)
        comp = r.integers(0, components, size=count)
        out = np.empty((count, dim), dtype=np.float32)
        step = 1 << 16
        for s in range(0, count, step):
            e = min(count, s + step)
            z = r.standard_normal(size=(e - s, dim), dtype=np.float32)
            out[s:e] = np.maximum(0.0, np.rint(means[comp[s:e]] + sigma * z))
        return out

    return draw(n, 1), draw(nq, 2)


def normalized_mixture(n: int, nq: int, dim: int = 96, components: int = 1024, config: int = 3):
    """C3 generator: unit-normalised mixture, queries perturbed from base points."""
    means = _rng(config, 0).standard_normal(size=(components, dim)).astype(np.float32)
    r = _rng(config, 1)
    comp = r.integers(0, components, size=n)
    base = means[comp] + 0.3 * r.standard_normal(size=(n, dim), dtype=np.float32)
    base /= np.linalg.norm(base, axis=1, keepdims=True)
    rq = _rng(config, 2)
    pick = rq.integers(0, n, size=nq)
    q = base[pick] + 0.05 * rq.standard_normal(size=(nq, dim), dtype=np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return base.astype(np.float32), q.astype(np.float32)


def unit_box_mixture(n: int, nq: int, dim: int = 960, components: int = 256, config: int = 4):
    """C4 generator: values in [0,1]."""
    means = _rng(config, 0).uniform(0.0, 1.0, size=(components, dim)).astype(np.float32)

    def draw(count: int, stream: int) -> np.ndarray:
        r = _rng(config, stream)
        comp = r.integers(0, components, size=count)
        z = r.standard_normal(size=(count, dim), dtype=np.float32)
        return np.clip(means[comp] + 0.1 * z, 0.0, 1.0).astype(np.float32)

    return draw(n, 1), draw(nq, 2)


def anisotropic_unit_mixture(n: int, nq: int, dim: int = 1536, components: int = 4096, config: int = 5):
    """C5 generator: unit-normalised anisotropic mixture (each component has
    its own per-dimension spread), queries drawn from the same mixture."""
    r0 = _rng(config, 0)
    means = r0.standard_normal(size=(components, dim)).astype(np.float32)
    scales = (0.05 + 0.45 * r0.uniform(0.0, 1.0, size=(components, dim))).astype(np.float32)

    def draw(count: int, stream: int) -> np.ndarray:
        r = _rng(config, stream)
        comp = r.integers(0, components, size=count)
        out = np.empty((count, dim), dtype=np.float32)
        step = 1 << 14
        for s in range(0, count, step):
            e = min(count, s + step)
            z = r.standard_normal(size=(e - s, dim), dtype=np.float32)
            x = means[comp[s:e]] + scales[comp[s:e]] * z
            out[s:e] = x / np.linalg.norm(x, axis=1, keepdims=True)
        return out

    return draw(n, 1), draw(nq, 2)


def anisotropic_unit_mixture_device(n: int, nq: int, dim: int = 1536, components: int = 4096, config: int = 5,
                                    device="cuda", chunk: int = 1 << 19):
    """The C5 mixture drawn on a torch device, for sets too large to draw on
    the host (10M x 1536 is 61 GB): the same means and per-component scales
    as anisotropic_unit_mixture (numpy, stream 0), with the component choices
    and the normal draws from torch generators on `device` seeded with the
    same per-stream seeds.  Returns float32 tensors (base, queries) on
    `device`; deterministic for a given device type and torch version (the
    host generator's values differ)."""
    import torch
    r0 = _rng(config, 0)
    means = torch.as_tensor(r0.standard_normal(size=(components, dim)).astype(np.float32), device=device)
    scales = torch.as_tensor((0.05 + 0.45 * r0.uniform(0.0, 1.0, size=(components, dim))).astype(np.float32),
                             device=device)

    def draw(count: int, stream: int):
        g = torch.Generator(device=device)
        g.manual_seed(SEED_BASE + 16 * config + stream)
        comp = torch.randint(0, components, (count,), generator=g, device=device)
        out = torch.empty((count, dim), dtype=torch.float32, device=device)
        for s in range(0, count, chunk):
            e = min(count, s + chunk)
            z = torch.randn((e - s, dim), generator=g, device=device, dtype=torch.float32)
            c = comp[s:e]
            x = torch.addcmul(means[c], scales[c], z)
            out[s:e] = x / torch.linalg.vector_norm(x, dim=1, keepdim=True)
            del z, x
        return out

    return draw(n, 1), draw(nq, 2)


def signs_for(padded_dim: int, config: int = 1) -> np.ndarray:
    """The +-1 diagonal of the rotation P = H_B * diag(signs)."""
    r = _rng(config, 3)
    return np.where(r.integers(0, 2, size=padded_dim) == 1, 1.0, -1.0).astype(np.float32)
