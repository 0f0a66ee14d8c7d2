"""gehtp_attn_decode_noalloc (the allocation-free decode attention entry point) against
gehtp_attn_decode with a caller's workspace, through the C ABI: bit-identical outputs on
two calls in a row, the second with a smaller KV cache and fewer heads (the shared
scratch keeps the first call's contents), and a request beyond the fixed scratch is
refused before anything launches."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import from_dev, normal_f16, ptr, stream_ptr, to_dev

pytestmark = pytest.mark.gpu

HD = 128
SCALE = float(np.float16(1.0 / np.sqrt(128)))
GEHTP_E2BIG = -7
MAX_FLOATS = 1 << 20


def _ring(lib, dev, rng, n_kv, KVH, nslots):
    import torch
    kv_elems = KVH * HD
    state_bytes = nslots * kv_elems * 4
    ring = torch.zeros(state_bytes, dtype=torch.uint8, device=dev)
    ks, vs = normal_f16(rng, n_kv, kv_elems), normal_f16(rng, n_kv, kv_elems)
    assert lib.gehtp_kv_append(ptr(ring), state_bytes, ptr(to_dev(ks, dev)), ptr(to_dev(vs, dev)), kv_elems, n_kv,
                               0, stream_ptr()) == 0
    return ring, state_bytes


def test_attn_decode_noalloc_matches_workspace_entry(lib, torch_dev):
    import torch
    rng = np.random.default_rng(77)
    outs = []
    for n_kv, H, KVH in ((4096, 32, 8), (300, 16, 8)):   # second call smaller
        ring, state_bytes = _ring(lib, torch_dev, rng, n_kv, KVH, 4096)
        q = to_dev(normal_f16(rng, H, HD), torch_dev)
        wf = lib.gehtp_attn_decode_work_floats(n_kv, H, HD)
        assert wf <= MAX_FLOATS
        work = torch.full((wf,), float("nan"), dtype=torch.float32, device=torch_dev)
        want = torch.empty((H, HD), dtype=torch.float16, device=torch_dev)
        got = torch.full((H, HD), float("nan"), dtype=torch.float16, device=torch_dev)
        assert lib.gehtp_attn_decode(ptr(q), ptr(ring), state_bytes, ptr(want), n_kv, H, KVH, HD, SCALE, ptr(work),
                                     wf, stream_ptr()) == 0
        assert lib.gehtp_attn_decode_noalloc(ptr(q), ptr(ring), state_bytes, ptr(got), n_kv, H, KVH, HD, SCALE,
                                             stream_ptr()) == 0
        torch.cuda.synchronize()
        a, b = from_dev(want), from_dev(got)
        assert np.isfinite(a.astype(np.float32)).all()
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"n_kv={n_kv} H={H}: outputs differ"
        outs.append(b)
    assert outs[0].shape != outs[1].shape


def test_attn_decode_noalloc_rejects_beyond_scratch(lib, torch_dev):
    """n_kv = 15936 at H = 32 needs 249 chunks of partials, one more than the scratch
    holds (15872 keys fit): refused with GEHTP_E2BIG, the output left untouched."""
    import torch
    H, KVH, nslots = 32, 8, 16384
    assert lib.gehtp_attn_decode_work_floats(15872, H, HD) <= MAX_FLOATS
    assert lib.gehtp_attn_decode_work_floats(15936, H, HD) > MAX_FLOATS
    state_bytes = nslots * KVH * HD * 4
    ring = torch.zeros(state_bytes, dtype=torch.uint8, device=torch_dev)
    q = torch.zeros((H, HD), dtype=torch.float16, device=torch_dev)
    out = torch.full((H, HD), 7.0, dtype=torch.float16, device=torch_dev)
    rc = lib.gehtp_attn_decode_noalloc(ptr(q), ptr(ring), state_bytes, ptr(out), 15936, H, KVH, HD, SCALE,
                                       stream_ptr())
    assert rc == GEHTP_E2BIG
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
