"""Prefill W4A16 GEMMs at the 4B-class model's own shapes (M = 2048
prompt tokens), unit-scale inputs, against the oracle: the fused q|k|v GEMM, gate/up with
the SwiGLU epilogue (N = 2 x 9728 interleaved rows), and the o- / down-projections with
the residual epilogue, which split K in three through an fp32 workspace (K = 4096, 9728),
also followed by the split's finishing pass that writes the next GEMM's RMSNorm rows.

Tolerance (written here because these outputs are not unit-sized): the BASELINE bar is
max-abs-err 2e-2 and cosine >= 0.9999 for unit-scale fp16 outputs. The GEMMs sum K =
2560 .. 9728 products, so outputs reach |y| ~ 10-60 where one fp16 ulp is 0.008-0.03;
any summation order other than the oracle's sequential k moves some of them by an ulp.
Each element must therefore satisfy |got - ref| <= 2e-2 * max(1, s), s the magnitude
at the last rounding (|ref|, or |acc| + |res| when a residual is added, since a sum that
cancels keeps the error of its larger operand); the whole output cosine >= 0.9999; and
at least 97 % of outputs equal the oracle's within one fp16 ulp.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import cosine, from_dev, normal_f16, ptr, stream_ptr, to_dev, w4g_weights

pytestmark = pytest.mark.gpu

M = 2048


def _sync():
    import torch
    torch.cuda.synchronize()


def _ulps(a, b):
    ai = a.view(np.int16).astype(np.int32)
    bi = b.view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def _check(got, ref, scale, what):
    g, r = got.astype(np.float64), ref.astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite"
    err = np.abs(g - r)
    bound = 2e-2 * np.maximum(1.0, scale)
    worst = int(np.argmax(err / bound))
    assert (err <= bound).all(), f"{what}: |err| {err.flat[worst]:.4g} at |scale| {scale.flat[worst]:.4g}"
    c = cosine(g, r)
    assert c >= 0.9999, f"{what}: cos {c:.7f}"
    within1 = float((_ulps(got, ref) <= 1).mean())
    assert within1 >= 0.97, f"{what}: only {within1:.4f} within one ulp"
    return c, within1


def _fused(lib, dev, x, wq, ws, N, K, mode=0, res=None, work=None):
    import torch
    n_out = N // 2 if mode else N
    y = torch.empty((M, n_out), dtype=torch.float16, device=dev)
    need = lib.gehtp_w4g_split_bytes(M, N, K)
    wk = torch.empty(max(need // 4, 1), dtype=torch.float32, device=dev) if work else None
    rc = lib.gehtp_w4g_fused_ws(ptr(to_dev(x, dev)), K, ptr(to_dev(wq, dev)), ptr(to_dev(ws, dev)), ptr(y), n_out,
                                M, N, K, None, ptr(to_dev(res, dev)) if res is not None else None, n_out, mode,
                                ptr(wk) if wk is not None else None, need if wk is not None else 0, stream_ptr())
    assert rc == 0, rc
    _sync()
    return from_dev(y), need


def test_qkv_gemm_4b(lib, oracle, torch_dev):
    rng = np.random.default_rng(501)
    N, K = 6144, 2560
    _, wq, ws = w4g_weights(rng, N, K)
    x = normal_f16(rng, M, K)
    got, _ = _fused(lib, torch_dev, x, wq, ws, N, K)
    ref = oracle.matmul_w4g(x, wq, ws, threads=16)
    _check(got, ref, np.abs(ref.astype(np.float64)), "qkv 2048x6144x2560")


def test_gate_up_swiglu_gemm_4b(lib, oracle, torch_dev):
    """gate/up rows interleaved (2j gate, 2j+1 up), SwiGLU epilogue: output column j =
    f16(f16(silu(f16(g))) * f16(u)) as UNARY silu then BINARY mul."""
    rng = np.random.default_rng(502)
    N, K = 2 * 9728, 2560
    _, wq, ws = w4g_weights(rng, N, K)
    x = normal_f16(rng, M, K)
    got, _ = _fused(lib, torch_dev, x, wq, ws, N, K, mode=1)
    acc = oracle.matmul_w4g(x, wq, ws, threads=16)
    ref = oracle.binary(oracle.unary(np.ascontiguousarray(acc[:, 0::2]), 12), np.ascontiguousarray(acc[:, 1::2]), 2)
    _check(got, ref, np.abs(ref.astype(np.float64)), "gate/up swiglu 2048x19456x2560")


@pytest.mark.parametrize("K", [4096, 9728])
def test_split_k_residual_gemm_4b(lib, oracle, torch_dev, K):
    """o-proj (K = 4096) and down-proj (K = 9728) at N = 2560 with the residual epilogue:
    the K-split path (workspace given) and the one-pass path, both against the oracle."""
    rng = np.random.default_rng(503 + K)
    N = 2560
    _, wq, ws = w4g_weights(rng, N, K)
    x = normal_f16(rng, M, K)
    res = normal_f16(rng, M, N)
    split, need = _fused(lib, torch_dev, x, wq, ws, N, K, res=res, work=True)
    assert need > 0, "this shape is expected to split K"
    one, _ = _fused(lib, torch_dev, x, wq, ws, N, K, res=res, work=False)
    acc = oracle.matmul_w4g(x, wq, ws, threads=16)
    ref = oracle.binary(acc, res, 0)
    scale = np.abs(acc.astype(np.float64)) + np.abs(res.astype(np.float64))
    _check(split, ref, scale, f"split-K residual K={K}")
    _check(one, ref, scale, f"one-pass residual K={K}")
