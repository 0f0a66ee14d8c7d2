"""Pins of the oracle's remaining runlist ops (crouton16_row4 surfaces, opcode 1/2,
concat/split/reduce/pad/cumsum/gather/transpose): each is checked against an
independent formulation (numpy's own array ops, closed forms, special cases)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import normal_f16


def _inv_crouton_by_decomposition(surf, M, K):
    """The surface index decomposition written out in kernels/host/inv_crouton16.py:
    pair p -> col_in_tile = p % 32, row_pair, m32_group, kt, row4_phase (innermost first)."""
    n_m32, n_kt = M // 32, K // 32
    pair = np.arange(M * K // 2)
    col_in_tile = pair % 32
    rest = pair // 32
    row_pair = rest % 2
    rest //= 2
    g = rest % n_m32
    rest //= n_m32
    kt = rest % n_kt
    phase = rest // n_kt
    row0 = g * 32 + phase * 4 + row_pair * 2
    col = kt * 32 + col_in_tile
    out = np.empty((M, K), np.uint16)
    out[row0, col] = surf[0::2]
    out[row0 + 1, col] = surf[1::2]
    return out


@pytest.mark.parametrize("M,K", [(32, 32), (64, 96), (256, 256), (96, 2560)])
def test_crouton_matches_index_decomposition(oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    lin = rng.integers(0, 65536, size=(M, K), dtype=np.uint16)
    surf = oracle.crouton_encode(lin)
    assert np.array_equal(_inv_crouton_by_decomposition(surf, M, K), lin)
    assert np.array_equal(oracle.crouton_decode(surf, M, K), lin)
    # the surface is a permutation: every element appears once
    assert np.array_equal(np.sort(surf), np.sort(lin.ravel()))


def test_crouton_first_block_layout(oracle):
    """The first 64 surface words: rows 0/1 of column 0..31 pair-interleaved
    (pos = 2*col + row) - kernels/docs/data_layout.md:40 pair-interleave."""
    M, K = 64, 64
    lin = (np.arange(M)[:, None] * 1000 + np.arange(K)[None, :]).astype(np.uint16)
    surf = oracle.crouton_encode(lin)
    assert list(surf[:6]) == [0, 1000, 1, 1001, 2, 1002]
    assert list(surf[64:66]) == [2000, 3000]        # row pair 1 (rows 2, 3) of group 0
    assert list(surf[128:130]) == [32000, 33000]    # group 1 (rows 32, 33)
    with pytest.raises(ValueError):
        oracle.crouton_encode(np.zeros((48, 64), np.uint16))


def _round_div7(s):
    """Nearest integer to s/7 via floor((2s + 7) / 14) (s/7 is never a tie)."""
    return (2 * s + 7) // 14


def _w4a16_numpy(A, W, M, K, N):
    s = (A.astype(np.int64) - 32768) @ W.astype(np.int64).T      # [M, N]
    return np.clip(_round_div7(s) + 32768, 0, 65535).astype(np.uint16)


@pytest.mark.parametrize("M,K,N", [(32, 32, 32), (64, 128, 96), (256, 256, 64)])
def test_matmul_w4a16_closed_form(oracle, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = rng.integers(0, 65536, size=(M, K), dtype=np.uint16)
    W = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    got = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(A), oracle.w4a16_pack(W), M, K, N), M, N)
    assert np.array_equal(got, _w4a16_numpy(A, W, M, K, N))


def test_matmul_w4a16_special_cases(oracle):
    M = K = N = 32
    rng = np.random.default_rng(3)
    zero = np.full((M, K), 32768, np.uint16)
    W = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    pack = oracle.w4a16_pack(W)
    y = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(zero), pack, M, K, N), M, N)
    assert (y == 32768).all()                                   # A' = 0 -> offset only
    # one-hot W (only k=5, value q): y = nearest((A[:,5]-32768) * q / 7) + 32768
    for q in (-8, -3, 1, 7):
        Wq = np.zeros((N, K), np.int8)
        Wq[:, 5] = q
        A = rng.integers(20000, 45000, size=(M, K), dtype=np.uint16)
        y = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(A), oracle.w4a16_pack(Wq), M, K, N), M, N)
        ref = np.array([[int(round((int(a) - 32768) * q / 7)) + 32768 for _ in range(N)] for a in A[:, 5]])
        assert np.array_equal(y.astype(np.int64), ref)
    # sign symmetry: A' -> -A' maps Y to 65536 - Y when nothing clips
    A = rng.integers(32768 - 400, 32768 + 400, size=(M, K), dtype=np.uint16)
    Aneg = (65536 - A.astype(np.int64)).astype(np.uint16)
    y1 = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(A), pack, M, K, N), M, N).astype(np.int64)
    y2 = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(Aneg), pack, M, K, N), M, N).astype(np.int64)
    assert np.array_equal(y1 + y2, np.full_like(y1, 65536))
    # clipping at both ends
    big = np.full((M, K), 65535, np.uint16)
    Wmax = np.full((N, K), 7, np.int8)
    Wmin = np.full((N, K), -8, np.int8)
    hi = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(big), oracle.w4a16_pack(Wmax), M, K, N), M, N)
    lo = oracle.crouton_decode(oracle.matmul_w4a16(oracle.crouton_encode(big), oracle.w4a16_pack(Wmin), M, K, N), M, N)
    assert (hi == 65535).all() and (lo == 0).all()


def test_rmsnorm_crouton_special_cases(oracle):
    m, n = 64, 64
    rng = np.random.default_rng(9)
    w = rng.uniform(0.5, 1.5, n).astype(np.float16)
    # zero rows (u16 32768) -> 0; constant rows c -> f16(c / sqrt(c^2 + 1e-6) * w)
    lin = np.full((m, n), 32768, np.uint16)
    consts = rng.integers(-30000, 30000, size=m // 2)
    for r, c in enumerate(consts):
        lin[2 * r] = 32768 + c
    y = oracle.rmsnorm_crouton(oracle.crouton_encode(lin), w, m, n)
    assert (y[1::2] == 0).all()
    for r, c in enumerate(consts):
        ref = (c / np.sqrt(float(c) ** 2 + 1e-6) * w.astype(np.float64)).astype(np.float16)
        ulps = np.abs(y[2 * r].view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
        assert ulps.max() <= 1, (c, ulps.max())
    with pytest.raises(ValueError):
        oracle.rmsnorm_crouton(np.zeros(48 * 64, np.uint16), w, 48, 64)


def test_rmsnorm_crouton_matches_float64(oracle):
    m, n = 96, 256
    rng = np.random.default_rng(10)
    lin = rng.integers(0, 65536, size=(m, n), dtype=np.uint16)
    w = rng.uniform(0.5, 1.5, n).astype(np.float16)
    y = oracle.rmsnorm_crouton(oracle.crouton_encode(lin), w, m, n).astype(np.float64)
    x = lin.astype(np.float64) - 32768
    ref = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.allclose(y, ref, rtol=2e-3, atol=1e-3)


def test_concat_split_round_trip(oracle):
    rng = np.random.default_rng(11)
    outer, sizes = 7, [3, 16, 5, 8]
    segs = [normal_f16(rng, outer, s) for s in sizes]
    y = oracle.concat(segs, outer).reshape(outer, -1)
    assert np.array_equal(y.view(np.uint16), np.concatenate(segs, axis=1).view(np.uint16))
    for k in range(4):
        back = oracle.split(y, sizes, k).reshape(outer, sizes[k])
        assert np.array_equal(back.view(np.uint16), segs[k].view(np.uint16))


@pytest.mark.parametrize("dims,axis", [([1, 1, 6, 40], 3), ([1, 3, 7, 5], 2), ([2, 9, 4, 3], 1), ([5, 2, 3, 4], 0)])
def test_reduce_against_numpy(oracle, dims, axis):
    rng = np.random.default_rng(sum(dims) + axis)
    # small integers: every f32 partial sum is exact, so the order cannot matter
    x = rng.integers(-8, 9, size=dims).astype(np.float16)
    for sub, fn in ((0, np.sum), (2, np.max), (3, np.min)):
        got = oracle.reduce(x, dims, axis, sub)
        ref = fn(x.astype(np.float64), axis=axis).astype(np.float16).ravel()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), sub
    # mean of a constant vector is that constant
    c = np.full(dims, 1.375, np.float16)
    assert (oracle.reduce(c, dims, axis, 1) == np.float16(1.375)).all()
    with pytest.raises(ValueError):
        oracle.reduce(x, dims, 4, 0)


def test_pad_against_numpy(oracle):
    rng = np.random.default_rng(12)
    x = normal_f16(rng, 5, 7)
    y = oracle.pad(x, 5, 7, 12, 3, -1.5).reshape(5, 12)
    ref = np.pad(x, ((0, 0), (3, 2)), constant_values=np.float16(-1.5))
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("exclusive,reverse", [(False, False), (True, False), (False, True), (True, True)])
def test_cumsum_against_numpy(oracle, exclusive, reverse):
    rng = np.random.default_rng(13)
    rows, n = 4, 33
    x = rng.integers(-5, 6, size=(rows, n)).astype(np.float16)
    got = oracle.cumsum(x, rows, n, exclusive, reverse).reshape(rows, n)
    v = x[:, ::-1] if reverse else x
    c = np.cumsum(v.astype(np.float64), axis=1)
    if exclusive:
        c = np.concatenate([np.zeros((rows, 1)), c[:, :-1]], axis=1)
    if reverse:
        c = c[:, ::-1]
    assert np.array_equal(got.astype(np.float64), c)


@pytest.mark.parametrize("td,xd,axis", [([10, 6], [4], 0), ([3, 10, 4], [2, 3], 1), ([6, 5], [7], 1)])
def test_gather_against_numpy_take(oracle, td, xd, axis):
    rng = np.random.default_rng(sum(td) + sum(xd) + axis)
    tbl = normal_f16(rng, *td)
    idx = rng.integers(-td[axis], td[axis], size=xd).astype(np.int32)
    got = oracle.gather(tbl, idx, td, xd, axis)
    ref = np.take(tbl, idx, axis=axis)            # negative indices wrap once, as the reference
    assert np.array_equal(got.view(np.uint16), ref.ravel().view(np.uint16))
    # out of range (after one wrap) gives zero
    bad = np.full(xd, td[axis], np.int32)
    assert (oracle.gather(tbl, bad, td, xd, axis) == 0).all()


@pytest.mark.parametrize("perm", [(0, 1, 2, 3), (0, 3, 1, 2), (0, 2, 3, 1), (0, 3, 2, 1)])
def test_transpose4_against_numpy(oracle, perm):
    rng = np.random.default_rng(14)
    Hh, W, Cc = 3, 5, 4
    x = normal_f16(rng, 1, Hh, W, Cc)
    got = oracle.transpose4(x, Hh, W, Cc, perm)
    ref = np.transpose(x, perm).ravel()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
