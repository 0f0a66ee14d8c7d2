"""Seeded inputs of the BASELINE configurations and the parity metrics."""
from __future__ import annotations

import numpy as np

# Parity bar for fp16 outputs: max-abs-err and cosine.
MAX_ABS = 2e-2
MIN_COS = 0.9999


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def assert_close(got, ref, max_abs=MAX_ABS, min_cos=MIN_COS, what=""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = float(np.max(np.abs(got - ref))) if got.size else 0.0
    cos = cosine(got, ref)
    assert err <= max_abs and cos >= min_cos, f"{what}: max_abs_err={err:.3g} cos={cos:.6f}"
    return err, cos


def w4g_weights(rng, N: int, K: int, smin=0.005, smax=0.02):
    """int4 q ~ U{-8..7}, fp16 scales ~ U[smin, smax] per group of 64."""
    from oracle import oracle as o
    q = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(smin, smax, size=(N, K // 64)).astype(np.float16)
    return q, o.w4g_pack(q), ws


def normal_f16(rng, *shape):
    return rng.standard_normal(shape).astype(np.float16)


# ---- torch plumbing (GPU tests only) ----
# Device tensors made by to_dev stay referenced until the test ends (conftest clears
# this list), so `ptr(to_dev(x))` inside a call cannot hand a kernel freed memory that
# the caching allocator gives to the next operand.
KEEP_ALIVE: list = []


def to_dev(a, dev):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        t = torch.from_numpy(a.view(np.int16)).to(dev).view(torch.float16)
    else:
        t = torch.from_numpy(a).to(dev)
    KEEP_ALIVE.append(t)
    return t


def from_dev(t) -> np.ndarray:
    import torch
    t = t.detach()
    if t.dtype == torch.float16:
        return t.view(torch.int16).cpu().numpy().view(np.float16)
    return t.cpu().numpy()


def stream_ptr():
    import torch
    return torch.cuda.current_stream().cuda_stream


def ptr(t) -> int:
    return t.data_ptr()
