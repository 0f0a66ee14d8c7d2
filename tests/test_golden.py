"""Committed fixtures (tests/golden/) against the oracle and the library's parser.
ref_* fixtures were produced by the reference's own C sources (see make_golden.py), so
these checks hold on machines without the reference tree."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from gehtp_amd.abi import WtBlob

G = Path(__file__).resolve().parent / "golden"


def test_softmax_host_form_matches_reference_fixture(oracle):
    d = np.load(G / "ref_softmax_host.npz")
    got = oracle.softmax(d["x"], 8, 256, form="host")
    assert np.array_equal(got.view(np.uint16), d["y_f16"].view(np.uint16))
    # the dispatch form picks the host variant for n % 32 == 0
    assert np.array_equal(oracle.softmax(d["x"], 8, 256).view(np.uint16), d["y_f16"].view(np.uint16))


def test_kv_ring_matches_reference_fixture(oracle):
    d = np.load(G / "ref_kvcache.npz")
    ring = oracle.KVRing(int(d["nslots"]) * int(d["kv_elems"]) * 4, int(d["kv_elems"]))
    for i, p in enumerate(d["pos"]):
        assert ring.append(d["k"][i], d["v"][i], int(p)) == d["slots"][i]
    assert np.array_equal(ring.buf, d["ring"])
    assert np.array_equal(ring.posmap, d["posmap"])


def test_parser_matches_reference_fixture(lib):
    d = np.load(G / "ref_parse.npz")
    data, lens, codes = d["data"].tobytes(), d["lens"], d["codes"]
    off = 0
    assert codes[0] == 0 and (codes != 0).any()
    for n, code in zip(lens, codes):
        b = data[off:off + int(n)]
        off += int(n)
        buf = C.create_string_buffer(b, len(b))
        assert lib.wt_parse(C.cast(buf, C.POINTER(C.c_uint8)), len(b), C.byref(WtBlob())) == code


def test_w4g_oracle_fixture(oracle):
    d = np.load(G / "oracle_w4g_small.npz")
    K = d["x"].shape[1]
    assert np.array_equal(oracle.w4g_dequant(d["wq"], d["ws"], K).view(np.uint16), d["w"].view(np.uint16))
    assert np.array_equal(oracle.matmul_w4g(d["x"], d["wq"], d["ws"]).view(np.uint16), d["y"].view(np.uint16))


def test_e2e_fixture_order_band():
    """The config-5 fixture carries, per row, the order-only band (largest top-64 move
    when the oracle sums in its two other fp32 orders) and each order's own leader: the
    band is positive and below the logits' scale, and wherever the golden margin exceeds
    twice the band both other orders pick the golden top-1 (the property the GPU gate's
    tie rule rests on)."""
    import numpy as np
    from pathlib import Path
    fx = np.load(Path(__file__).resolve().parent / "golden" / "e2e_4b_seed0.npz")
    band, top2, am, alt = fx["band"], fx["top2"], fx["argmax"], fx["alt_argmax"]
    assert list(fx["orders"]) == [1, 2] and alt.shape == (2, len(am))
    assert (band > 0).all() and (band < 0.02 * np.abs(top2[:, 0])).all()
    margin = top2[:, 0] - top2[:, 1]
    clear = margin > 2 * band
    assert clear.sum() >= len(am) - 6
    assert (alt[:, clear] == am[clear]).all()
