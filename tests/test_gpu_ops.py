"""GPU parity of the remaining runlist ops against the CPU oracle: crouton16_row4
surfaces, OP_MATMUL_W4A16 (opcode 1), OP_RMSNORM_F16 (opcode 2), and the data ops
(FILL, TRANSPOSE, CONCAT, SPLIT, REDUCE, CUMSUM, GATHER, DMA, PAD) through the engine.
Integer and data-movement results are bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import from_dev, normal_f16, ptr, stream_ptr, to_dev

from gehtp_amd.abi import opcodes as OP
from gehtp_amd.runlist import BlobBuilder

pytestmark = pytest.mark.gpu

DMA_FENCE_NONE = 0xFF
REF_VTCM = 0x4000
REF_ENG = 0xC000
ENG_OUT = 1


def _sync():
    import torch
    torch.cuda.synchronize()


@pytest.fixture(autouse=True)
def fresh_engine(engine, torch_dev):
    engine.shutdown()
    engine.state_reset()
    yield
    engine.shutdown()


# ---------------------------------------------------------------- kernels ----
@pytest.mark.parametrize("rows,cols", [(32, 32), (96, 64), (256, 2560)])
def test_crouton_encode_decode(lib, oracle, torch_dev, rows, cols):
    import torch
    rng = np.random.default_rng(rows + cols)
    lin = rng.integers(0, 65536, size=(rows, cols), dtype=np.uint16)
    ld = to_dev(lin.view(np.int16), torch_dev)
    surf = torch.empty(rows * cols, dtype=torch.int16, device=torch_dev)
    assert lib.gehtp_crouton_encode(ptr(ld), ptr(surf), rows, cols, stream_ptr()) == 0
    back = torch.empty_like(ld)
    assert lib.gehtp_crouton_decode(ptr(surf), ptr(back), rows, cols, stream_ptr()) == 0
    _sync()
    assert np.array_equal(surf.cpu().numpy().view(np.uint16), oracle.crouton_encode(lin))
    assert np.array_equal(back.cpu().numpy().view(np.uint16), lin)
    assert lib.gehtp_crouton_encode(ptr(ld), ptr(surf), 48, cols, stream_ptr()) != 0


@pytest.mark.parametrize("M,K,N", [(32, 32, 32), (96, 160, 64), (256, 2560, 2560)])
def test_matmul_w4a16_bit_exact(lib, oracle, torch_dev, M, K, N):
    """Opcode 1 at the reference's s2560 shape (M=256, K=N=2560) and small shapes."""
    import torch
    rng = np.random.default_rng(M * 3 + K + N)
    A = rng.integers(0, 65536, size=(M, K), dtype=np.uint16)
    W = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    act = oracle.crouton_encode(A)
    wslot = oracle.w4a16_pack(W)
    out = torch.empty(M * N, dtype=torch.int16, device=torch_dev)
    assert lib.gehtp_matmul_w4a16(ptr(to_dev(act.view(np.int16), torch_dev)), ptr(to_dev(wslot, torch_dev)), ptr(out),
                                  M, K, N, stream_ptr()) == 0
    _sync()
    ref = oracle.matmul_w4a16(act, wslot, M, K, N)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref)


def test_matmul_w4a16_extremes(lib, oracle, torch_dev):
    """All-max activations against all -8 / +7 weights: clipping at 0 and 65535, and
    the int64 accumulation across K steps."""
    import torch
    M, K, N = 64, 4096, 64
    for a_val, w_val in ((65535, 7), (65535, -8), (0, 7), (0, -8)):
        A = np.full((M, K), a_val, np.uint16)
        W = np.full((N, K), w_val, np.int8)
        act, wslot = oracle.crouton_encode(A), oracle.w4a16_pack(W)
        out = torch.empty(M * N, dtype=torch.int16, device=torch_dev)
        assert lib.gehtp_matmul_w4a16(ptr(to_dev(act.view(np.int16), torch_dev)), ptr(to_dev(wslot, torch_dev)),
                                      ptr(out), M, K, N, stream_ptr()) == 0
        _sync()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), oracle.matmul_w4a16(act, wslot, M, K, N))


@pytest.mark.parametrize("m,n", [(32, 64), (256, 2560)])
def test_rmsnorm_crouton(lib, oracle, torch_dev, m, n):
    import torch
    rng = np.random.default_rng(m + n)
    lin = rng.integers(0, 65536, size=(m, n), dtype=np.uint16)
    lin[3] = 32768                                   # a zero row
    w = rng.uniform(0.5, 1.5, n).astype(np.float16)
    surf = oracle.crouton_encode(lin)
    y = torch.empty((m, n), dtype=torch.float16, device=torch_dev)
    assert lib.gehtp_rmsnorm_crouton(ptr(to_dev(surf.view(np.int16), torch_dev)), ptr(to_dev(w, torch_dev)), ptr(y),
                                     m, n, stream_ptr()) == 0
    _sync()
    ref = oracle.rmsnorm_crouton(surf, w, m, n)
    ulps = np.abs(from_dev(y).view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.999      # double sum order may flip one ulp


# ---------------------------------------------------------------- engine -----
def _w4_blob(M, K, N, act, wslot, rms_w, dma: bool):
    """The reference's pack_oplist.cc blob shapes: w5 (MATMUL from the act slot, then
    RMSNORM on its output) or w4dma (act DMA'd into a VTCM temp, MATMUL in place, the
    engine's out surface DMA'd to temp 0, then RMSNORM)."""
    bb = BlobBuilder()
    s_act = bb.add_slot(act.view(np.uint8))
    s_w = bb.add_slot(wslot)
    bb.add_slot(np.zeros((N // 32) * 512, np.uint8))            # folded bias
    bb.add_slot(np.arange(8 * (K // 32), dtype=np.uint32))      # act table
    bb.add_slot(np.arange(8 * (K // 32), dtype=np.uint32))      # out table
    s_rms = bb.add_slot(rms_w)
    act_b = M * K * 2
    bb.op(OP.NOP)
    bb.op(OP.PIN, s_w)
    bb.op(OP.PIN, 2)
    if dma:
        st = 9
        bb.set_tempoff(2 * M * N * 2, [(0, 0, M * N * 2), (1, M * N * 2, M * N * 2), (REF_VTCM | st, 0, act_b)],
                       bump_kb=128, vtcm_kb=(act_b + 1023) // 1024)
        bb.op(OP.DMA, 0x8000 | s_act, REF_VTCM | st, act_b, 0, 0, 1, 0, 2)
        bb.op(OP.MATMUL_W4A16, REF_VTCM | st, s_w, 0, M, K, N)
        bb.op(OP.DMA, REF_ENG | ENG_OUT, 0, M * N * 2, 0, 0, 1, 2, 0)
    else:
        bb.op(OP.MATMUL_W4A16, s_act, s_w, 0, M, K, N)
    bb.op(OP.RMSNORM_F16, 0, s_rms, 1, N)
    return bb.build()


@pytest.mark.parametrize("dma", [False, True])
def test_engine_w4a16_rmsnorm_blob(engine, oracle, dma):
    M, K, N = 256, 2560, 2560
    rng = np.random.default_rng(5 + dma)
    A = rng.integers(0, 65536, size=(M, K), dtype=np.uint16)
    W = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    act, wslot = oracle.crouton_encode(A), oracle.w4a16_pack(W)
    rms_w = (1.0 + 0.3 * np.sin(0.37 * np.arange(N))).astype(np.float16)
    pb = engine.parse(_w4_blob(M, K, N, act, wslot, rms_w, dma))
    m, _ = engine.run(pb)
    assert m == M                                   # engine_m reports the W4A16 engine's M
    y_ref = oracle.matmul_w4a16(act, wslot, M, K, N)
    assert np.array_equal(np.frombuffer(engine.temp(0), np.uint16), y_ref)
    z = np.frombuffer(engine.temp(1), np.float16).reshape(M, N)
    z_ref = oracle.rmsnorm_crouton(y_ref, rms_w, M, N)
    ulps = np.abs(z.view(np.int16).astype(np.int32) - z_ref.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1
    assert engine.stats().matmul == 1 and engine.stats().rmsnorm == 1


def test_engine_w4a16_errors(engine, oracle):
    """Reference error behaviour: missing supply slots, wrong act / weight slot sizes."""
    from gehtp_amd import WtExecError
    M, K, N = 32, 64, 64
    A = np.zeros((M, K), np.uint16)
    bb = BlobBuilder()
    s_act = bb.add_slot(oracle.crouton_encode(A).view(np.uint8))
    s_w = bb.add_slot(np.zeros(K * N // 2, np.uint8))
    bb.op(OP.MATMUL_W4A16, s_act, s_w, 0, M, K, N)
    with pytest.raises(WtExecError, match="supply slots missing"):
        engine.run(engine.parse(bb.build()))
    bb2 = BlobBuilder()
    s_act = bb2.add_slot(np.zeros(M * K * 2 - 128, np.uint8))
    s_w = bb2.add_slot(np.zeros(K * N // 2, np.uint8))
    bb2.add_slot(np.zeros((N // 32) * 512, np.uint8))
    bb2.add_slot(np.zeros(8 * (K // 32) * 4, np.uint8))
    bb2.add_slot(np.zeros(8 * (K // 32) * 4, np.uint8))
    bb2.op(OP.MATMUL_W4A16, s_act, s_w, 0, M, K, N)
    with pytest.raises(WtExecError, match="act slot size mismatch"):
        engine.run(engine.parse(bb2.build()))


@pytest.mark.parametrize("nz_byte", [0, 1, 2 * 512 - 1])
def test_engine_w4a16_nonzero_folded_bias_fails(engine, oracle, nz_byte):
    """The folded bias term of opcode 1 (+ bias_fold[n], kernels/docs/api_v22_w4a16.md:11)
    lives in the HMX engine's own (N/32) x 512-byte packing, which no readable source
    defines: a non-zero bias slot fails the op (first op, error names the slot), and the
    same blob with the bias zeroed runs and matches the oracle."""
    from gehtp_amd import WtExecError
    M, K, N = 32, 64, 64
    rng = np.random.default_rng(nz_byte)
    A = rng.integers(0, 65536, size=(M, K), dtype=np.uint16)
    W = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    act, wslot = oracle.crouton_encode(A), oracle.w4a16_pack(W)
    for nonzero in (True, False):
        bias = np.zeros((N // 32) * 512, np.uint8)
        if nonzero:
            bias[nz_byte] = 1
        bb = BlobBuilder()
        s_act = bb.add_slot(act.view(np.uint8))
        s_w = bb.add_slot(wslot)
        s_b = bb.add_slot(bias)
        bb.add_slot(np.zeros(8 * (K // 32) * 4, np.uint8))
        bb.add_slot(np.zeros(8 * (K // 32) * 4, np.uint8))
        bb.op(OP.MATMUL_W4A16, s_act, s_w, 0, M, K, N)
        pb = engine.parse(bb.build())
        if nonzero:
            with pytest.raises(WtExecError, match=f"folded bias slot {s_b} is non-zero"):
                engine.run(pb)
        else:
            engine.run(pb)
            assert np.array_equal(np.frombuffer(engine.temp(0), np.uint16), oracle.matmul_w4a16(act, wslot, M, K, N))


def test_engine_data_ops(engine, oracle):
    """FILL, TRANSPOSE, CONCAT, SPLIT, REDUCE, CUMSUM, GATHER, PAD and DMA in one runlist,
    each output temp bit-exact against the oracle."""
    rng = np.random.default_rng(21)
    bb = BlobBuilder()
    pool = normal_f16(rng, 300)
    s_pool = bb.add_slot(pool)
    x = normal_f16(rng, 1, 3, 5, 8)                       # (1, H, W, C)
    s_x = bb.add_slot(x)
    segs = [normal_f16(rng, 6, s) for s in (4, 12, 8)]
    s_segs = [bb.add_slot(g) for g in segs]
    red = rng.integers(-8, 9, size=(2, 3, 4, 5)).astype(np.float16)
    s_red = bb.add_slot(red)
    tbl = normal_f16(rng, 10, 6)
    s_tbl = bb.add_slot(tbl)
    idx = rng.integers(-10, 12, size=(4,)).astype(np.int32)
    s_idx = bb.add_slot(idx)
    T = {k: bb.temp() for k in ("fill", "tr", "cat", "spl", "red", "cum", "gat", "pad", "dma")}
    bb.op(OP.FILL, s_pool, 20, T["fill"], 100)
    bb.op(OP.TRANSPOSE_F16, 0x8000 | s_x, T["tr"], 3, 5, 8, 0 | (3 << 8) | (1 << 16) | (2 << 24))
    total = 4 + 12 + 8
    bb.op(OP.CONCAT_F16, *[0x8000 | s for s in s_segs], 0, 0, 0, 0, 0, T["cat"], 0, 3, 6 * total, 4, 12, 8, 0)
    bb.op(OP.SPLIT_F16, T["cat"], T["spl"], 0, 0, 0, 0, 0, 0, 0, 0, 3, 4, 12, 8, 0, 1)
    bb.op(OP.REDUCE_F16, 0x8000 | s_red, T["red"], red.size, 2, 0, 2, 3, 4, 5)
    bb.op(OP.CUMSUM_F32, 0x8000 | s_red, T["cum"], 6, 20, 0, 1, 1)
    bb.op(OP.GATHER_F16, 0x8000 | s_tbl, 0x8000 | s_idx, T["gat"], 4 * 6, 0 | (1 << 8) | (2 << 16),
          10, 6, 1, 1, 1, 4, 1, 1, 1, 1)
    bb.op(OP.PAD_F16, T["fill"], T["pad"], 10, 10, 16, 2, int(np.float16(-2.5).view(np.uint16)))
    bb.op(OP.DMA, T["pad"], T["dma"], 64, 32, 8, 1, DMA_FENCE_NONE, DMA_FENCE_NONE)
    engine.run(engine.parse(bb.build()))

    def got(name, n):
        return np.frombuffer(engine.temp(T[name]), np.uint16)[:n]

    assert np.array_equal(got("fill", 100), pool[10:110].view(np.uint16))
    assert np.array_equal(got("tr", x.size), oracle.transpose4(x, 3, 5, 8, (0, 3, 1, 2)).view(np.uint16))
    cat = oracle.concat(segs, 6)
    assert np.array_equal(got("cat", cat.size), cat.view(np.uint16))
    spl = oracle.split(cat, [4, 12, 8], 1)
    assert np.array_equal(got("spl", spl.size), spl.view(np.uint16))
    r = oracle.reduce(red, [2, 3, 4, 5], 2, 0)
    assert np.array_equal(got("red", r.size), r.view(np.uint16))
    c = oracle.cumsum(red, 6, 20, True, True)
    assert np.array_equal(got("cum", c.size), c.view(np.uint16))
    gth = oracle.gather(tbl, idx, [10, 6], [4], 0)
    assert np.array_equal(got("gat", gth.size), gth.view(np.uint16))
    pd = oracle.pad(pool[10:110], 10, 10, 16, 2, -2.5)
    assert np.array_equal(got("pad", pd.size), pd.view(np.uint16))
    dma = np.frombuffer(engine.temp(T["dma"]), np.uint8)[8:8 + 64]
    assert np.array_equal(dma, pd.view(np.uint8)[32:96])
