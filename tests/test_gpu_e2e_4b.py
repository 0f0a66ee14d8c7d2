"""BASELINE config 5 end to end: the 4B-class Qwen3-style W4A16 runlist (36 layers, hidden
2560, 32 Q / 8 KV heads at head_dim 128, FFN 9728, vocab 151936 fp16 lm_head), a prompt
of 2048 seeded token ids, then 256 greedy decode steps, through the engine's C ABI.

Checked against the CPU golden (tests/golden/e2e_4b_seed0.npz, written by
tests/golden/make_e2e_4b.py from the oracle's restatement of the reference runlist), with
the reference's own decode gate (scripts/judge_logits.py:1-30: cosine >= 0.9999 and the
same top-1):
  - the prompt's last-token logits and every decode step the fixture holds: cosine
    >= 0.9999 over every 8th logit, and the 64 largest logits within max(2e-2, 1 % of
    |ref|) of the oracle's;
  - top-1: the fixture also holds, per step, the order-only band: how far the oracle's
    own logits move (largest change over the 64 leaders) when its fp32 sums run in two
    other valid orders with the same roundings (32-wide slices combined pairwise, the
    decode GEMV's shape; 16-deep slices added in sequence, the GEMM's K steps). Two
    leaders each moving by up to the band can swap only when their golden margin is at
    most twice it, so wherever the margin exceeds twice the band the engine's top-1
    must be the golden's, with no allowance; at the remaining steps (ties at the
    precision fixed by the summation order, not by the engine) it must be one of the
    golden leaders within twice the band of the first. Every such step is reported with
    its margin and band;
  - the decode steps are teacher forced: the engine consumes the fixture's ids, which are
    the oracle's own greedy choices, so with top-1 identical it runs the same greedy path;
  - every one of the 256 steps: finite logits, and the token the blob's ARGMAX op returns
    is the first maximum of those logits;
  - the same prompt and 256 steps run again with the engine's graph replay off give the
    same bits at every step (the first run captures the decode step into a HIP graph on
    its second identical run and replays it afterwards).
"""
from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest

from helpers import cosine

pytestmark = pytest.mark.gpu

FIX = Path(__file__).resolve().parent / "golden" / "e2e_4b_seed0.npz"
STEPS = 256


def _image_crc(img: np.ndarray) -> int:
    crc = 0
    step = 1 << 26
    for o in range(0, img.size, step):
        crc = zlib.crc32(img[o:o + step], crc)
    return crc


@pytest.fixture(scope="module")
def model4b():
    from gehtp_amd.qwen3 import CONFIG_4B, Weights, emit_decode, emit_prefill
    fx = dict(np.load(FIX))
    w = Weights(CONFIG_4B, seed=int(fx["seed"]))
    assert _image_crc(w.image) == int(fx["image_crc"]), "weight image differs from the fixture's"
    S = int(fx["prompt"])
    max_pos = S + STEPS + 64
    pre, tp = emit_prefill(CONFIG_4B, w, S, max_pos)
    dec, td = emit_decode(CONFIG_4B, w, max_pos)
    return CONFIG_4B, w, fx, pre, tp, dec, td


def _generate(engine, model, graphs: bool):
    """Prompt + STEPS greedy steps; the first steps consume the fixture's ids. Returns the
    logits rows (fp16, row 0 = prompt) and the tokens the ARGMAX op returned."""
    cfg, w, fx, pre, tp, dec, td = model
    prev = engine.set_graphs(graphs)
    try:
        engine.shutdown()
        engine.set_ext_weights(w.image.ctypes.data)
        pp, pd = engine.parse(pre), engine.parse(dec)
        engine.state_reset()
        emb = w.embed()
        out, _ = engine.run_io(pp, np.ascontiguousarray(emb[fx["prompt_ids"]]).tobytes(), tp["tok"])
        rows = [np.frombuffer(engine.temp(tp["logits"]), np.float16)[:cfg.vocab].copy()]
        toks = [int(np.frombuffer(out, np.int32)[0])]
        forced = fx["decode_ids"]
        for t in range(STEPS):
            nxt = int(forced[t]) if t < len(forced) else toks[-1]
            out, _ = engine.run_io(pd, emb[nxt].tobytes(), td["tok"])
            rows.append(np.frombuffer(engine.temp(td["logits"]), np.float16)[:cfg.vocab].copy())
            toks.append(int(np.frombuffer(out, np.int32)[0]))
        engine.shutdown()
    finally:
        engine.set_graphs(prev)
    return rows, toks


def test_config5_e2e_vs_cpu_golden(engine, model4b):
    cfg, w, fx, *_ = model4b
    c0, r0 = engine.graph_stats()
    rows, toks = _generate(engine, model4b, graphs=True)
    c1, r1 = engine.graph_stats()
    assert r1 - r0 >= STEPS - 8, f"decode steps were not replayed from a graph ({c1 - c0} captured, {r1 - r0} replays)"

    for t, (row, tok) in enumerate(zip(rows, toks)):
        f = row.astype(np.float32)
        assert np.isfinite(f).all(), f"step {t}: non-finite logits"
        assert tok == int(np.argmax(f)), f"step {t}: ARGMAX op gave {tok}, logits' first max {int(np.argmax(f))}"

    stride = int(fx["stride"])
    band = fx["band"].astype(np.float64)
    assert band.shape == (len(fx["argmax"]),) and (band > 0).all(), "fixture without its order-only band"
    margins, worst_rel, exact, ties, ratio = [], 0.0, 0, [], []
    for t in range(len(fx["argmax"])):
        g = rows[t].astype(np.float32)
        want = int(fx["argmax"][t])
        top2 = fx["top2"][t]
        margin = float(top2[0] - top2[1])
        margins.append(margin)
        c = cosine(g[::stride], fx["logits_strided"][t].astype(np.float32))
        assert c >= 0.9999, f"step {t}: cos {c:.6f} over every {stride}th logit"
        ti, tv = fx["top_idx"][t], fx["top_val"][t].astype(np.float64)
        tol = np.maximum(2e-2, 1e-2 * np.abs(tv))
        err = np.abs(g[ti].astype(np.float64) - tv)
        assert (err <= tol).all(), f"step {t}: top-64 logit off by {err.max():.4g}"
        worst_rel = max(worst_rel, float((err / np.maximum(np.abs(tv), 1e-3)).max()))
        ratio.append(float(err.max()) / band[t])
        tie = 2.0 * band[t]
        got = int(np.argmax(g))
        if margin > tie:
            assert got == want, (f"step {t}: top-1 {got} vs golden {want} at a golden margin of {margin:.4g}, "
                                 f"above twice the order-only band ({tie:.4g})")
            exact += 1
        else:
            cand = {int(i) for i, v in zip(ti, tv) if v >= tv[0] - tie}
            assert got in cand, f"step {t}: tie (margin {margin:.4g} <= {tie:.4g}), top-1 {got} not in {cand}"
            ties.append((t, round(margin, 4), round(float(band[t]), 4), got == want))
    print(f"config 5: {exact} of {len(margins)} golden rows above twice the order-only band, all top-1 "
          f"identical; ties within it (step, margin, band, same top-1): {ties}; margins min {min(margins):.4g} "
          f"median {float(np.median(margins)):.4g}; engine top-64 error / band: max {max(ratio):.3g} median "
          f"{float(np.median(ratio)):.3g}; top-64 worst relative error {worst_rel:.3g}; {STEPS} greedy steps")

    direct, dtoks = _generate(engine, model4b, graphs=False)
    assert dtoks == toks
    for t, (a, b) in enumerate(zip(rows, direct)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {t}: graph replay and direct runs differ"


def test_config5_with_a_static_temp_plan(engine, model4b):
    """The 36-layer model's prefill (2048 tokens) and 8 decode steps with a TEMPOFF static
    plan (the SwiGLU activation sharing bytes with the attention tensors) give the bits of
    the bump-allocated blobs at every step."""
    from gehtp_amd.qwen3 import CONFIG_4B, emit_decode, emit_prefill
    cfg, w, fx, pre, tp, dec, td = model4b
    S, max_pos = int(fx["prompt"]), int(fx["prompt"]) + STEPS + 64
    pre2, tp2 = emit_prefill(CONFIG_4B, w, S, max_pos, tempoff=True)
    dec2, td2 = emit_decode(CONFIG_4B, w, max_pos, tempoff=True)
    emb = w.embed()
    runs = []
    for (p_, tp_, d_, td_) in ((pre, tp, dec, td), (pre2, tp2, dec2, td2)):
        engine.shutdown()
        engine.set_ext_weights(w.image.ctypes.data)
        pp, pd = engine.parse(p_), engine.parse(d_)
        engine.state_reset()
        engine.run_io(pp, np.ascontiguousarray(emb[fx["prompt_ids"]]).tobytes(), tp_["tok"])
        rows = [np.frombuffer(engine.temp(tp_["logits"]), np.float16)[:cfg.vocab].copy()]
        for t in range(8):
            engine.run_io(pd, emb[int(fx["decode_ids"][t])].tobytes(), td_["tok"])
            rows.append(np.frombuffer(engine.temp(td_["logits"]), np.float16)[:cfg.vocab].copy())
        engine.shutdown()
        runs.append(rows)
    for t, (a, b) in enumerate(zip(*runs)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {t}"
