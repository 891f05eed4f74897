"""Memory layouts the element-wise step can run over in storage order."""
from __future__ import annotations

import torch


def dense_layout(t: torch.Tensor) -> bool:
    """Whether t's elements fill one gap-free, non-overlapping block of
    memory in some order (contiguous, or a permutation of it such as a
    transposed matrix): then an element-wise update can run over its
    numel() elements from data_ptr() on.  Dimensions of size 1 are ignored,
    and an empty tensor (whatever its strides) has nothing to lay out."""
    if t.numel() == 0:
        return True
    dims = sorted((st, n) for n, st in zip(t.shape, t.stride()) if n != 1)
    expect = 1
    for st, n in dims:
        if st != expect:
            return False
        expect *= n
    return True


def no_overlap(t: torch.Tensor) -> bool:
    """Whether t's elements are known to sit at distinct addresses: ordered by
    stride, each dimension of size > 1 steps past the whole extent of the
    smaller ones (contiguous, permuted and sliced layouts such as
    ``x[:, :k]`` or ``x[::2]``).  An expanded tensor (stride 0) fails, as
    does any layout this rule cannot clear."""
    if t.numel() == 0:
        return True
    extent = 0
    for st, n in sorted((st, n) for n, st in zip(t.shape, t.stride()) if n != 1):
        if st <= extent:
            return False
        extent += st * (n - 1)
    return True


def same_layout(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same shape and the same strides on every dimension of size > 1 (any
    strides, for empty tensors)."""
    return a.shape == b.shape and (a.numel() == 0 or all(n == 1 or sa == sb for n, sa, sb in zip(a.shape, a.stride(), b.stride())))
