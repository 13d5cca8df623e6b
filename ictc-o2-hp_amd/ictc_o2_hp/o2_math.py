"""Real Cartesian O(2) coupling coefficients, built once on the host in fp64.

This is the coefficient source of the product: every table the HIP kernels use
is derived from the functions below when a module is constructed.  The
construction follows ``src/ictc_o2_hp/o2_math.py`` of Parity-LRX/ICTC-O2-HP:

* harmonic polynomials of frequency m are Re/Im of (x + i y)^m written in the
  monomial basis x^a y^(m-a), orthonormalised under the O(2)-invariant
  Gaussian Gram matrix (``o2_math.py:42-53``, ``:86-134``);
* the SO(2) coupling of frequencies (m1, m2) into m3 multiplies the two
  harmonic polynomials and projects onto the frequency-m3 harmonic lifted by
  (x^2 + y^2)^k (``o2_math.py:144-157``, ``:242-280``);
* the O(2) rules add the even/odd scalars and the J intertwiner used for the
  reflection-odd scalar (``o2_math.py:282-346``) and the admissible output keys
  (``o2_math.py:348-372``).

Arithmetic is numpy float64.  The public functions return torch tensors with
the reference's names and signatures so code written against the reference's
``o2_math`` keeps working.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache
from typing import Dict, List, Tuple

import numpy as np
import torch

O2IrrepKey = Tuple[str, int]

_J = np.array([[0.0, -1.0], [1.0, 0.0]])


def so2_irrep_dim(m: int) -> int:
    """1 for the frequency-0 scalar, 2 for every positive frequency."""
    m = int(m)
    if m < 0:
        raise ValueError(f"frequency m must be >= 0, got {m}")
    return 1 if m == 0 else 2


def _monomials(degree: int) -> List[Tuple[int, int]]:
    """Exponents (a, b) of x^a y^b with a + b = degree, a ascending."""
    if degree < 0:
        raise ValueError(f"L must be >= 0, got {degree}")
    return [(a, degree - a) for a in range(degree + 1)]


def _odd_double_factorial(n: int) -> int:
    result = 1
    while n > 1:
        result *= n
        n -= 2
    return result


def _gaussian_moment(n: int) -> float:
    """E[t^n] for t ~ N(0, 1): (n-1)!! for even n, 0 for odd n."""
    return 0.0 if n % 2 else float(_odd_double_factorial(n - 1))


@lru_cache(maxsize=None)
def _gram(degree: int) -> np.ndarray:
    """Gaussian inner products of the degree-L monomials (``o2_math.py:42-53``)."""
    mons = _monomials(degree)
    return np.array([[_gaussian_moment(a + c) * _gaussian_moment(b + d)
                      for (c, d) in mons] for (a, b) in mons])


@lru_cache(maxsize=None)
def _radial_lift(degree: int, k: int) -> np.ndarray:
    """Matrix of multiplication by (x^2 + y^2)^k (``o2_math.py:55-74``)."""
    if degree < 0 or k < 0:
        raise ValueError(f"L_src and k must be >= 0, got {degree}, {k}")
    target = {mon: row for row, mon in enumerate(_monomials(degree + 2 * k))}
    lift = np.zeros((degree + 2 * k + 1, degree + 1))
    for col, (a, b) in enumerate(_monomials(degree)):
        for q in range(k + 1):
            lift[target[(a + 2 * q, b + 2 * (k - q))], col] += math.comb(k, q)
    return lift


def _first_nonzero_positive(vector: np.ndarray) -> np.ndarray:
    """Flip the sign so the first entry above 1e-12 is positive (``o2_math.py:76-84``)."""
    for value in vector:
        if abs(value) > 1e-12:
            return -vector if value < 0.0 else vector
    return vector


@lru_cache(maxsize=None)
def _harmonic_basis(m: int) -> np.ndarray:
    """Monomial coefficients of the frequency-m harmonics, shape (m+1, dim).

    Columns are the cos and sin members; see ``o2_math.py:86-134`` for the
    conventions (Gram-Schmidt order, sign fix, negated cos for even m).
    """
    m = int(m)
    if m < 0:
        raise ValueError(f"m must be >= 0, got {m}")
    if m == 0:
        return np.ones((1, 1))
    # i^b for b = 0..3 split into real and imaginary parts.
    re_phase = (1.0, 0.0, -1.0, 0.0)
    im_phase = (0.0, 1.0, 0.0, -1.0)
    cos_vec = np.array([math.comb(m, a) * re_phase[b % 4] for a, b in _monomials(m)])
    sin_vec = np.array([math.comb(m, a) * im_phase[b % 4] for a, b in _monomials(m)])
    gram = _gram(m)
    cos_vec = cos_vec / math.sqrt(max(float(cos_vec @ gram @ cos_vec), 1e-30))
    sin_vec = sin_vec - float(cos_vec @ gram @ sin_vec) * cos_vec
    sin_vec = sin_vec / math.sqrt(max(float(sin_vec @ gram @ sin_vec), 1e-30))
    cos_vec = _first_nonzero_positive(cos_vec)
    sin_vec = _first_nonzero_positive(sin_vec)
    if m % 2 == 0:
        cos_vec = -cos_vec
    return np.stack([cos_vec, sin_vec], axis=-1)


@lru_cache(maxsize=None)
def _projector(degree: int, m: int) -> np.ndarray:
    """Coefficients of the r^(2k)-lifted frequency-m harmonic in a degree-L
    polynomial, L = m + 2k: (V^T G V)^-1 V^T G (``o2_math.py:144-157``)."""
    k = (degree - m) // 2
    lifted = _radial_lift(m, k) @ _harmonic_basis(m)
    gram = _gram(degree)
    return np.linalg.solve(lifted.T @ gram @ lifted, lifted.T @ gram)


@lru_cache(maxsize=None)
def _product_matrix(m1: int, m2: int) -> np.ndarray:
    """Polynomial multiplication of degree-m1 by degree-m2 monomials (``o2_math.py:242-254``)."""
    target = {mon: row for row, mon in enumerate(_monomials(m1 + m2))}
    second = _monomials(m2)
    out = np.zeros((m1 + m2 + 1, (m1 + 1) * (m2 + 1)))
    for i, (a1, b1) in enumerate(_monomials(m1)):
        for j, (a2, b2) in enumerate(second):
            out[target[(a1 + a2, b1 + b2)], i * len(second) + j] = 1.0
    return out


@lru_cache(maxsize=None)
def _so2_coupling(m1: int, m2: int, m3: int) -> np.ndarray:
    """SO(2) coupling tensor C[i, j, k] in the real [cos, sin] bases (``o2_math.py:256-280``)."""
    d1, d2, d3 = so2_irrep_dim(m1), so2_irrep_dim(m2), so2_irrep_dim(m3)
    if min(m1, m2, m3) < 0:
        raise ValueError(f"m1, m2, m3 must be >= 0, got {(m1, m2, m3)}")
    if m3 > m1 + m2 or (m1 + m2 + m3) % 2:
        return np.zeros((d1, d2, d3))
    b1, b2 = _harmonic_basis(m1), _harmonic_basis(m2)
    # Each (i, j) basis product as a degree-(m1+m2) polynomial, then its
    # frequency-m3 coordinates.
    products = np.einsum("pi,qj->pqij", b1, b2).reshape(b1.shape[0] * b2.shape[0], d1 * d2)
    coords = _projector(m1 + m2, m3) @ (_product_matrix(m1, m2) @ products)
    return coords.T.reshape(d1, d2, d3).copy()


def _normalize_key(key) -> O2IrrepKey:
    """Accept ("scalar", +-1), ("freq", m>=1) or the tokens "0e", "0o", "m"."""
    if isinstance(key, tuple):
        tag, value = key
        tag = str(tag).strip().lower()
        value = int(value)
        if tag == "scalar" and value in (-1, 1):
            return ("scalar", value)
        if tag == "freq" and value >= 1:
            return ("freq", value)
        raise ValueError(f"Invalid O(2) key {key!r}")
    token = str(key).strip().lower()
    if token == "0e":
        return ("scalar", 1)
    if token == "0o":
        return ("scalar", -1)
    if token.isdigit() and int(token) >= 1:
        return ("freq", int(token))
    raise ValueError(f"Invalid O(2) irrep token {key!r}")


def key_dim(key) -> int:
    return 1 if _normalize_key(key)[0] == "scalar" else 2


def valid_output_keys(key1, key2) -> List[O2IrrepKey]:
    """Irreps in key1 (x) key2, in the reference's order (``o2_math.py:348-372``)."""
    k1, k2 = _normalize_key(key1), _normalize_key(key2)
    if k1[0] == "scalar" and k2[0] == "scalar":
        return [("scalar", k1[1] * k2[1])]
    if k1[0] == "scalar":
        return [k2]
    if k2[0] == "scalar":
        return [k1]
    m1, m2 = k1[1], k2[1]
    if m1 == m2:
        return [("scalar", 1), ("scalar", -1), ("freq", 2 * m1)]
    return [("freq", abs(m1 - m2)), ("freq", m1 + m2)]


@lru_cache(maxsize=None)
def cg_numpy(key1, key2, key3) -> np.ndarray:
    """Unnormalised O(2) coupling C[i, j, k] as float64 (``o2_math.py:295-346``)."""
    k1, k2, k3 = _normalize_key(key1), _normalize_key(key2), _normalize_key(key3)
    d1, d2, d3 = key_dim(k1), key_dim(k2), key_dim(k3)
    zero = np.zeros((d1, d2, d3))
    if k1[0] == "scalar" and k2[0] == "scalar":
        return np.ones((1, 1, 1)) if k3 == ("scalar", k1[1] * k2[1]) else zero
    if k1[0] == "scalar" or k2[0] == "scalar":
        freq, scalar = (k2, k1) if k1[0] == "scalar" else (k1, k2)
        if k3 != freq:
            return zero
        # Stored as C[input, output]; J^T makes the output J times the input,
        # which is what the reflection-odd scalar requires.
        inter = np.eye(2) if scalar[1] == 1 else _J.T.copy()
        return inter[None, :, :] if k1[0] == "scalar" else inter[:, None, :]
    m1, m2 = k1[1], k2[1]
    if k3[0] == "freq":
        return _so2_coupling(m1, m2, k3[1])
    if m1 != m2:
        return zero
    if k3 == ("scalar", 1):
        return _so2_coupling(m1, m2, 0)
    odd = np.zeros((2, 2, 1))
    odd[0, 1, 0], odd[1, 0, 0] = 1.0, -1.0
    return odd


def normalized_cg(key1, key2, key3, normalization: str = "component") -> np.ndarray:
    """Coupling scaled to Frobenius norm sqrt(dim(k3)) ("component") or 1
    ("norm"), as ``native_o2.py:118-123`` does per path."""
    cg = cg_numpy(_normalize_key(key1), _normalize_key(key2), _normalize_key(key3))
    norm = float(np.linalg.norm(cg))
    if norm > 1.0e-30:
        if normalization == "component":
            cg = cg * (math.sqrt(cg.shape[2]) / norm)
        elif normalization == "norm":
            cg = cg / norm
    return cg


# --- reference-compatible public names --------------------------------------

def o2_valid_output_keys(key1, key2) -> List[O2IrrepKey]:
    """Every O(2) irrep admitted by ``key1 (x) key2`` (``o2_math.py:159-167``)."""
    return valid_output_keys(key1, key2)


def o2_cg_tensor(key1, key2, key3, *, dtype=None, device=None) -> torch.Tensor:
    """Real Cartesian O(2) Clebsch-Gordan tensor (``o2_math.py:169-185``)."""
    out = torch.from_numpy(cg_numpy(_normalize_key(key1), _normalize_key(key2),
                                    _normalize_key(key3)).copy())
    if dtype is not None or device is not None:
        out = out.to(dtype=dtype, device=device)
    return out


@dataclass(frozen=True)
class HarmonicProjectors2D:
    """Frequency projectors of the degree-L Cartesian polynomials, L <= Lmax.

    ``P[(L, m)]`` (m = L, L-2, ..., shape (dim(m), L+1), float64) maps the
    monomial coefficients of a degree-L polynomial to its coordinates on the
    frequency-m harmonics lifted by (x^2 + y^2)^((L-m)/2), orthogonally under
    the Gaussian Gram matrix (``o2_math.py:140-157``)."""
    Lmax: int
    P: Dict[Tuple[int, int], torch.Tensor]


@lru_cache(maxsize=None)
def build_harmonic_projectors_2d(Lmax: int) -> HarmonicProjectors2D:
    """All projectors ``P[(L, m)]`` for 0 <= L <= Lmax (``o2_math.py:144-157``)."""
    Lmax = int(Lmax)
    table = {(L, L - 2 * k): torch.from_numpy(_projector(L, L - 2 * k).copy())
             for L in range(Lmax + 1) for k in range(L // 2 + 1)}
    return HarmonicProjectors2D(Lmax=Lmax, P=table)


def build_cg_tensor_so2(m1: int, m2: int, m3: int) -> torch.Tensor:
    """SO(2) coupling in the real [cos, sin] basis (``o2_math.py:256-280``)."""
    return torch.from_numpy(_so2_coupling(int(m1), int(m2), int(m3)).copy())


def o2_representation(g: torch.Tensor, key) -> torch.Tensor:
    """Representation matrices of batched O(2) elements ``g`` (..., 2, 2).

    Frequency m uses [[cos m t, -det sin m t], [sin m t, det cos m t]]; the odd
    scalar is det(g) (``o2_math.py:187-216``).
    """
    k = _normalize_key(key)
    if g.shape[-2:] != (2, 2):
        raise ValueError(f"g must end with (2, 2), got {tuple(g.shape)}")
    det = torch.linalg.det(g)
    if k[0] == "scalar":
        value = torch.ones_like(det) if k[1] == 1 else det
        return value[..., None, None]
    angle = torch.atan2(g[..., 1, 0], g[..., 0, 0]) * float(k[1])
    c, s = torch.cos(angle), torch.sin(angle)
    return torch.stack((torch.stack((c, -det * s), -1), torch.stack((s, det * c), -1)), -2)

