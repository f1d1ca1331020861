"""Strided views over device buffers: how graph values map onto HBM without copies.

A value is a view (buffer, element offset, dims, element strides). transpose permutes strides; reshape re-strides
when numpy could (contiguous runs split or merged), so the reference's layout ops (anvil/interp/graph.py:76-81)
cost no kernel unless a consumer needs a dense layout the view does not have.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import hostpar

ITEMSIZE = {"i8": 1, "i16": 2, "i32": 4}


class Buf:
    """A planned device allocation (bytes); `mem` is the DeviceBuffer once allocated."""
    __slots__ = ("nbytes", "mem", "name")

    def __init__(self, nbytes: int, name: str = ""):
        self.nbytes, self.mem, self.name = int(nbytes), None, name

    @property
    def ptr(self) -> int:
        return self.mem.ptr


def contig_strides(dims) -> tuple:
    st, acc = [], 1
    for d in reversed(list(dims)):
        st.append(acc)
        acc *= int(d)
    return tuple(reversed(st))


@dataclass
class View:
    buf: Buf
    dtype: str
    dims: tuple
    strides: tuple
    offset: int = 0
    # K-blocked storage of the last dim (0: none): element (..., r, k) at the lead offset + (k // 64) * kb + k % 64,
    # the row stride (strides[-2]) being 64 -- the layout of ANVIL_GEMM_*_KBLOCK operands, read only by GEMMs
    kb: int = 0

    @property
    def itemsize(self) -> int:
        return ITEMSIZE[self.dtype]

    @property
    def size(self) -> int:
        return math.prod(self.dims)

    @property
    def ptr(self) -> int:
        return self.buf.ptr + self.offset * self.itemsize

    def is_contiguous(self) -> bool:
        if self.kb:
            return False
        return all(s == c for d, s, c in zip(self.dims, self.strides, contig_strides(self.dims)) if d != 1)

    def permute(self, perm) -> "View":
        if self.kb and list(perm)[-1] != len(self.dims) - 1:
            raise ValueError("a K-blocked view keeps its last dim last")
        return View(self.buf, self.dtype, tuple(self.dims[p] for p in perm), tuple(self.strides[p] for p in perm),
                    self.offset, self.kb)

    def reshape(self, newdims):
        """The same elements as `newdims` in row-major order, or None when that needs a copy."""
        if self.kb:                                   # lead dims only: the blocked last dim stays as it is,
            newdims = tuple(int(d) for d in newdims)  # or splits into its 64-element blocks (a plain view)
            if len(newdims) >= 2 and newdims[-1] == 64 and newdims[-2] * 64 == self.dims[-1]:
                st = nocopy_strides(self.dims[:-1], self.strides[:-1], newdims[:-2])
                return None if st is None else View(self.buf, self.dtype, newdims, (*st, self.kb, 1), self.offset)
            if not newdims or newdims[-1] != self.dims[-1]:
                return None
            st = nocopy_strides(self.dims[:-1], self.strides[:-1], newdims[:-1])
            return None if st is None else View(self.buf, self.dtype, tuple(newdims), (*st, 1), self.offset, self.kb)
        st = nocopy_strides(self.dims, self.strides, newdims)
        return None if st is None else View(self.buf, self.dtype, tuple(newdims), st, self.offset)

    def merge_kblocked(self, newdims):
        """A plain view whose last two dims are (n, 64) with strides (kb, 1), presented as newdims (..., n * 64) in
        K-blocked storage of block stride kb: the inverse of splitting a K-blocked last dim into its blocks. None when
        the view is not of that form or its lead dims do not reshape without a copy."""
        newdims = tuple(int(d) for d in newdims)
        if (self.kb or len(self.dims) < 2 or self.dims[-1] != 64 or self.strides[-1] != 1 or not newdims
                or newdims[-1] != self.dims[-2] * 64):
            return None
        st = nocopy_strides(self.dims[:-2], self.strides[:-2], newdims[:-1])
        return None if st is None else View(self.buf, self.dtype, newdims, (*st, 1), self.offset, self.strides[-2])

    def prepend(self, n: int) -> "View":
        """Broadcast over a new leading dim of size n (stride 0)."""
        return View(self.buf, self.dtype, (n,) + self.dims, (0,) + self.strides, self.offset, self.kb)

    def view(self, base: np.ndarray) -> np.ndarray:
        """This view of `base` (the whole buffer downloaded as self.dtype), at that dtype: without a copy, or for
        K-blocked storage a copy in the logical order (its 64-element blocks of a row are kb elements apart)."""
        isz = self.itemsize
        if self.kb:
            if self.dims[-1] % 64:
                raise ValueError("K-blocked storage holds whole 64-element blocks")
            blocks = np.lib.stride_tricks.as_strided(
                base[self.offset:], shape=(*self.dims[:-1], self.dims[-1] // 64, 64),
                strides=tuple(s * isz for s in self.strides[:-1]) + (self.kb * isz, isz))
            return blocks.reshape(self.dims)
        return np.lib.stride_tricks.as_strided(base[self.offset:], shape=self.dims,
                                               strides=tuple(s * isz for s in self.strides))

    def read(self, base: np.ndarray) -> np.ndarray:
        """This view of `base` as a new int64 array."""
        return hostpar.astype(self.view(base), np.int64)


def nocopy_strides(dims, strides, newdims):
    """Strides that present (dims, strides) as newdims without moving data, or None.

    The old dims are grouped into maximal runs whose strides nest (stride_i == stride_{i+1} dim_{i+1}); each new dim
    must fall inside one run, whose elements it then walks contiguously at the run's innermost stride."""
    dims, strides, newdims = list(map(int, dims)), list(map(int, strides)), list(map(int, newdims))
    if math.prod(dims) != math.prod(newdims):
        return None
    runs = []
    for d, s in zip(dims, strides):
        if d == 1:
            continue
        if runs and runs[-1][1] == s * d:
            runs[-1] = (runs[-1][0] * d, s)
        else:
            runs.append((d, s))
    out = [0] * len(newdims)
    idx = [i for i, d in enumerate(newdims) if d != 1]
    pos = 0
    for size, base in runs:
        group, prod = [], 1
        while prod < size and pos < len(idx):
            group.append(idx[pos])
            prod *= newdims[idx[pos]]
            pos += 1
        if prod != size:
            return None
        acc = base
        for i in reversed(group):
            out[i] = acc
            acc *= newdims[i]
    if pos != len(idx):
        return None
    return tuple(out)
