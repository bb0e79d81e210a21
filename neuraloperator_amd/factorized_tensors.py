"""Complex spectral-weight storage: dense and factorized (Tucker, CP, TT).

The reference stores SpectralConv weights in tensorly-torch 0.5.0
``FactorizedTensor`` objects (used at neuralop/layers/spectral_convolution.py
:362-370, read with ``.to_tensor()`` at :39-40, sliced at :489 and
contracted through ``.core``/``.factors`` at :101-103).  tltorch is not a
dependency here; these classes keep the parts of its behaviour the spectral
path relies on:

* ``FactorizedTensor.new(shape, rank, factorization, fixed_rank_modes, dtype)``
* ``.normal_(mean, std)``, ``.to_tensor()``, ``.name``, ``.shape``,
  ``.dtype``, ``.rank``
* slicing returns a factorized tensor of the window (mode factors are cut,
  the core is shared) -- tltorch's ``__getitem__`` semantics
* torch functions applied to one (``torch.is_complex(w)``) see the dense tensor

Rank rules (``rank`` given as a fraction) restate tensorly 0.9.0's
validate_*_rank; the resulting tuples are parity unpinned (tensorly cannot
be imported here).  Weights are complex64 ``nn.Parameter`` tensors; state-dict
keys are this package's own (``tensor`` / ``core`` + ``factors.i`` /
``weights`` + ``factors.i``).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

import torch
from torch import nn


def tucker_rank(shape: Sequence[int], rank, fixed_modes=None) -> List[int]:
    """Tucker ranks from a fraction of the dense parameter count (tensorly
    validate_tucker_rank, rounding='round')."""
    shape = list(shape)
    if isinstance(rank, (list, tuple)):
        return [int(r) for r in rank]
    if isinstance(rank, int) and not isinstance(rank, bool):
        return [rank] * len(shape)
    if rank == "same":
        rank = 1.0
    rank = float(rank)
    n_param = float(math.prod(shape))
    fixed = []
    work = list(shape)
    if fixed_modes:
        fixed = [(m, work.pop(m)) for m in sorted(fixed_modes, reverse=True)][::-1]
    n_fixed = float(sum(s * s for _, s in fixed))
    sq = float(sum(s * s for s in work))
    n_comp = len(work)

    def f(x):
        return n_param * x ** n_comp + sq * x + n_fixed * x - rank * n_param

    lo, hi = 0.0, max(rank, 1.0)
    for _ in range(200):
        mid = 0.5 * (lo + hi)
        if f(lo) * f(mid) <= 0:
            hi = mid
        else:
            lo = mid
    frac = 0.5 * (lo + hi)
    out = [max(int(round(s * frac)), 1) for s in work]
    for mode, size in fixed:
        out.insert(mode, size)
    return out


def cp_rank(shape: Sequence[int], rank) -> int:
    """tensorly validate_cp_rank for a fraction: round(rank * prod / sum)."""
    if isinstance(rank, int) and not isinstance(rank, bool):
        return rank
    if rank == "same":
        rank = 1.0
    return max(int(round(float(rank) * math.prod(shape) / sum(shape))), 1)


def tt_rank(shape: Sequence[int], rank) -> List[int]:
    """tensorly validate_tt_rank for a fraction (constant inner rank solving
    the parameter-count quadratic)."""
    n = len(shape)
    if isinstance(rank, (list, tuple)):
        return [int(r) for r in rank]
    if isinstance(rank, int) and not isinstance(rank, bool):
        return [1] + [rank] * (n - 1) + [1]
    if rank == "same":
        rank = 1.0
    n_param = float(math.prod(shape))
    a = float(sum(shape[1:-1]))
    b = float(shape[0] + shape[-1])
    c = -float(rank) * n_param
    if a == 0:
        r = max(int(round(-c / b)), 1)
    else:
        r = max(int(round((-b + math.sqrt(b * b - 4 * a * c)) / (2 * a))), 1)
    ranks = [1] + [r] * (n - 1) + [1]
    # a TT rank cannot exceed the matricization bounds
    for k in range(1, n):
        left = math.prod(shape[:k])
        right = math.prod(shape[k:])
        ranks[k] = min(ranks[k], left, right)
    return ranks


class FactorizedTensor(nn.Module):
    """Base of the complex weight containers."""

    name = "Base"

    @staticmethod
    def new(shape, rank=1.0, factorization="Dense", fixed_rank_modes=None, dtype=torch.cfloat,
            device=None, **kwargs):
        key = (factorization or "Dense").lower()
        if key.startswith("complex"):
            key = key[len("complex"):]
        if key == "dense":
            return DenseTensor(shape, dtype=dtype, device=device)
        if key == "tucker":
            return TuckerTensor(shape, tucker_rank(shape, rank, fixed_rank_modes), dtype=dtype,
                                device=device)
        if key == "cp":
            return CPTensor(shape, cp_rank(shape, rank), dtype=dtype, device=device)
        if key == "tt":
            return TTTensor(shape, tt_rank(shape, rank), dtype=dtype, device=device)
        raise ValueError(f"Got unexpected factorization {factorization}")

    @staticmethod
    def from_tensor(tensor, rank=None, factorization="ComplexDense"):
        """A weight container holding a copy of a full tensor (tltorch's
        FactorizedTensor.from_tensor, used as in the reference's
        test_spectral_convolution.py:52-55).  Only the dense form is built:
        decomposing into CP / Tucker / TT factors is not."""
        key = (factorization or "Dense").lower()
        if key.startswith("complex"):
            key = key[len("complex"):]
        if key != "dense":
            raise NotImplementedError(f"from_tensor into a {factorization} factorization is not built")
        return DenseTensor(tensor.shape, tensor=tensor.detach().clone())

    @property
    def dtype(self):
        return self.to_tensor().dtype

    def dim(self):
        return len(self.shape)

    @property
    def ndim(self):
        return len(self.shape)

    def size(self, d=None):
        return self.shape if d is None else self.shape[d]

    def __getitem__(self, idx):
        if not isinstance(idx, tuple):
            idx = (idx,)
        return self._slice(idx)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}

        def conv(a):
            if isinstance(a, FactorizedTensor):
                return a.to_tensor()
            if isinstance(a, (list, tuple)):
                return type(a)(conv(b) for b in a)
            return a

        return func(*conv(args), **{k: conv(v) for k, v in kwargs.items()})


def _complex_normal_(t: torch.Tensor, std: float):
    with torch.no_grad():
        t.normal_(0.0, std)  # complex normal_: real and imag each N(0, std^2/2)
    return t


class DenseTensor(FactorizedTensor):
    name = "ComplexDense"

    def __init__(self, shape, dtype=torch.cfloat, device=None, tensor: Optional[torch.Tensor] = None):
        super().__init__()
        if tensor is None:
            tensor = torch.empty(tuple(shape), dtype=dtype, device=device)
        self.tensor = nn.Parameter(tensor)
        self.rank = None

    @property
    def shape(self):
        return tuple(self.tensor.shape)

    def to_tensor(self):
        return self.tensor

    def normal_(self, mean=0.0, std=1.0):
        if mean != 0:
            raise ValueError(f"Currently only mean=0 is supported, but got mean={mean}")
        _complex_normal_(self.tensor, std)
        return self

    def _slice(self, idx):
        return _DenseView(self.tensor[idx])


class _DenseView(FactorizedTensor):
    """A window of a dense weight (shares storage; autograd flows to the parameter)."""
    name = "ComplexDense"

    def __init__(self, tensor):
        super().__init__()
        self._t = tensor
        self.rank = None

    @property
    def shape(self):
        return tuple(self._t.shape)

    def to_tensor(self):
        return self._t

    def _slice(self, idx):
        return _DenseView(self._t[idx])


class TuckerTensor(FactorizedTensor):
    """Tucker weight: W = core x_0 U_0 x_1 U_1 ... (U_d [shape_d, rank_d])."""
    name = "ComplexTucker"

    def __init__(self, shape, rank, dtype=torch.cfloat, device=None, core=None, factors=None):
        super().__init__()
        self._shape = tuple(shape)
        self.rank = tuple(rank)
        if core is None:
            core = torch.empty(self.rank, dtype=dtype, device=device)
        if factors is None:
            factors = [torch.empty((s, r), dtype=dtype, device=device) for s, r in zip(shape, rank)]
        self.core = nn.Parameter(core)
        self.factors = nn.ParameterList([nn.Parameter(f) for f in factors])

    @property
    def shape(self):
        return tuple(f.shape[0] for f in self.factors)

    @property
    def order(self):
        return len(self.rank)

    def to_tensor(self):
        t = self.core
        for mode, U in enumerate(self.factors):
            t = torch.movedim(torch.tensordot(t, U, dims=([mode], [1])), -1, mode)
        return t

    def normal_(self, mean=0.0, std=1.0):
        if mean != 0:
            raise ValueError(f"Currently only mean=0 is supported, but got mean={mean}")
        r = math.prod(math.sqrt(r) for r in self.rank)
        std_factors = (std / r) ** (1.0 / (self.order + 1))
        _complex_normal_(self.core, std_factors)
        for f in self.factors:
            _complex_normal_(f, std_factors)
        return self

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _TuckerView(self.core, [U[s] for U, s in zip(self.factors, idx)])


class _TuckerView(FactorizedTensor):
    name = "ComplexTucker"

    def __init__(self, core, factors):
        super().__init__()
        self.core = core
        self.factors = list(factors)
        self.rank = tuple(core.shape)

    @property
    def shape(self):
        return tuple(f.shape[0] for f in self.factors)

    def to_tensor(self):
        t = self.core
        for mode, U in enumerate(self.factors):
            t = torch.movedim(torch.tensordot(t, U, dims=([mode], [1])), -1, mode)
        return t

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _TuckerView(self.core, [U[s] for U, s in zip(self.factors, idx)])


class CPTensor(FactorizedTensor):
    """CP weight: W = sum_r w_r u_0r o u_1r o ... (U_d [shape_d, rank])."""
    name = "ComplexCP"

    def __init__(self, shape, rank, dtype=torch.cfloat, device=None, weights=None, factors=None):
        super().__init__()
        self.rank = int(rank)
        if weights is None:
            weights = torch.empty((self.rank,), dtype=dtype, device=device)
        if factors is None:
            factors = [torch.empty((s, self.rank), dtype=dtype, device=device) for s in shape]
        self.weights = nn.Parameter(weights)
        self.factors = nn.ParameterList([nn.Parameter(f) for f in factors])

    @property
    def shape(self):
        return tuple(f.shape[0] for f in self.factors)

    def to_tensor(self):
        return _cp_full(self.weights, list(self.factors))

    def normal_(self, mean=0.0, std=1.0):
        if mean != 0:
            raise ValueError(f"Currently only mean=0 is supported, but got mean={mean}")
        std_factors = (std / math.sqrt(self.rank)) ** (1.0 / len(self.factors))
        with torch.no_grad():
            self.weights.fill_(1.0)
        for f in self.factors:
            _complex_normal_(f, std_factors)
        return self

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _CPView(self.weights, [U[s] for U, s in zip(self.factors, idx)])


def _cp_full(weights, factors):
    syms = "abcdefghijklmnopqrstuvwxy"[: len(factors)]
    eq = "z," + ",".join(s + "z" for s in syms) + "->" + syms
    return torch.einsum(eq, weights, *factors)


class _CPView(FactorizedTensor):
    name = "ComplexCP"

    def __init__(self, weights, factors):
        super().__init__()
        self.weights = weights
        self.factors = list(factors)
        self.rank = weights.shape[0]

    @property
    def shape(self):
        return tuple(f.shape[0] for f in self.factors)

    def to_tensor(self):
        return _cp_full(self.weights, self.factors)

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _CPView(self.weights, [U[s] for U, s in zip(self.factors, idx)])


class TTTensor(FactorizedTensor):
    """Tensor-train weight: cores G_k [r_k, shape_k, r_{k+1}]."""
    name = "ComplexTT"

    def __init__(self, shape, rank, dtype=torch.cfloat, device=None, factors=None):
        super().__init__()
        self.rank = tuple(rank)
        if factors is None:
            factors = [torch.empty((rank[k], s, rank[k + 1]), dtype=dtype, device=device)
                       for k, s in enumerate(shape)]
        self.factors = nn.ParameterList([nn.Parameter(f) for f in factors])

    @property
    def shape(self):
        return tuple(f.shape[1] for f in self.factors)

    def to_tensor(self):
        return _tt_full(list(self.factors))

    def normal_(self, mean=0.0, std=1.0):
        if mean != 0:
            raise ValueError(f"Currently only mean=0 is supported, but got mean={mean}")
        r = math.prod(self.rank)
        std_factors = (std / math.sqrt(r)) ** (1.0 / len(self.factors))
        for f in self.factors:
            _complex_normal_(f, std_factors)
        return self

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _TTView([G[:, s, :] for G, s in zip(self.factors, idx)])


def _tt_full(factors):
    full = factors[0]
    for f in factors[1:]:
        full = torch.tensordot(full, f, dims=([-1], [0]))
    return full.squeeze(0).squeeze(-1)


class _TTView(FactorizedTensor):
    name = "ComplexTT"

    def __init__(self, factors):
        super().__init__()
        self.factors = list(factors)
        self.rank = tuple([f.shape[0] for f in factors] + [factors[-1].shape[-1]])

    @property
    def shape(self):
        return tuple(f.shape[1] for f in self.factors)

    def to_tensor(self):
        return _tt_full(self.factors)

    def _slice(self, idx):
        idx = tuple(idx) + (slice(None),) * (len(self.factors) - len(idx))
        return _TTView([G[:, s, :] for G, s in zip(self.factors, idx)])
