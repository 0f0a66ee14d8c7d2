"""Pins of the oracle's shape ops against numpy (CPU): OP_BROADCAST_F16, OP_TRANSPOSE_GEN_F16
and OP_STRIDED_SLICE_F16 restated from oplist_exec.c:1876-1988 must equal
numpy.broadcast_to / numpy.transpose / basic slicing on every shape numpy defines, so a
wrong stride, a dropped axis or a swapped permutation byte fails here."""
from __future__ import annotations

import itertools

import numpy as np
import pytest


def _x(rng, n):
    return rng.standard_normal(n).astype(np.float16)


@pytest.mark.parametrize("in_d,out_d", [
    ([1, 128], [4, 128]), ([1, 64], [8, 64]), ([5, 1, 8], [5, 3, 8]), ([2, 1, 3, 8], [2, 4, 3, 8]),
    ([3, 1], [3, 7]), ([1, 1, 6], [2, 5, 6]), ([4], [4]), ([1], [9]), ([2, 3, 1, 1], [2, 3, 1, 1]),
    ([7, 1, 1], [7, 2, 5]),
])
def test_broadcast_equals_numpy(oracle, in_d, out_d):
    rng = np.random.default_rng(len(in_d) * 10 + len(out_d))
    x = _x(rng, int(np.prod(in_d)))
    want = np.broadcast_to(x.reshape(in_d), out_d).ravel()
    got = oracle.broadcast(x, in_d, out_d)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("dims", [(3, 5), (4, 3, 8), (2, 3, 4, 5), (7, 1, 6)])
def test_transpose_gen_equals_numpy(oracle, dims):
    rng = np.random.default_rng(sum(dims))
    x = _x(rng, int(np.prod(dims)))
    for perm in itertools.permutations(range(len(dims))):
        want = np.transpose(x.reshape(dims), perm).ravel()
        got = oracle.transpose_gen(x, dims, perm)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), perm


@pytest.mark.parametrize("d,b,e,s", [
    ((40,), (3,), (37,), (1,)), ((40,), (1,), (40,), (2,)), ((40,), (0,), (40,), (7,)),
    ((6, 128), (0, 0), (6, 64), (1, 1)), ((6, 128), (0, 64), (6, 128), (1, 1)),
    ((5, 20), (0, 1), (5, 20), (1, 2)), ((5, 20), (1, 0), (5, 20), (2, 3)),
    ((3, 4, 10), (1, 0, 2), (3, 4, 9), (1, 2, 3)), ((4, 6, 8), (0, 1, 0), (4, 6, 8), (3, 1, 2)),
])
def test_slice_equals_numpy(oracle, d, b, e, s):
    rng = np.random.default_rng(sum(d))
    x = _x(rng, int(np.prod(d)))
    want = x.reshape(d)[tuple(slice(bb, ee, ss) for bb, ee, ss in zip(b, e, s))].ravel()
    got = oracle.strided_slice(x, want.size, b, e, s, d)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
