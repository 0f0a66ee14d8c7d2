"""End-to-end: Qwen3-style W4A16 runlists (gehtp_amd.qwen3) on the engine vs the oracle
model, teacher-forced: per step logits within tolerance and top-1 identical (the
reference's decode gate, scripts/judge_logits.py: cos >= 0.9999, exact top-1)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import cosine

from gehtp_amd.qwen3 import CONFIG_08B_LAYER, Qwen3Config, Weights, emit_decode, emit_prefill

pytestmark = pytest.mark.gpu

SMALL = Qwen3Config(layers=2, hidden=512, heads=4, kv_heads=2, ffn=1024, vocab=3000)


def _run(engine, cfg, S, n_dec, seed, max_pos=256, with_ref=True):
    from oracle.qwen3_ref import RefModel
    w = Weights(cfg, seed=seed)
    engine.shutdown()
    engine.set_ext_weights(w.image.ctypes.data)
    pre, tp = emit_prefill(cfg, w, S, max_pos)
    dec, td = emit_decode(cfg, w, max_pos)
    pp, pd = engine.parse(pre), engine.parse(dec)
    engine.state_reset()
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, cfg.vocab, S + n_dec)
    emb = w.embed()
    ref = RefModel(cfg, w, max_pos) if with_ref else None
    out, _ = engine.run_io(pp, np.ascontiguousarray(emb[ids[:S]]).tobytes(), tp["tok"])
    got = [np.frombuffer(engine.temp(tp["logits"]), np.float16)[:cfg.vocab].copy()]
    refl = [ref.prefill(np.ascontiguousarray(emb[ids[:S]]))] if ref else []
    assert int(np.frombuffer(out, np.int32)[0]) == int(np.argmax(got[0].astype(np.float32)))
    for t in range(n_dec):   # teacher forced: both sides consume ids[S + t]
        out, _ = engine.run_io(pd, emb[ids[S + t]].tobytes(), td["tok"])
        got.append(np.frombuffer(engine.temp(td["logits"]), np.float16)[:cfg.vocab].copy())
        assert int(np.frombuffer(out, np.int32)[0]) == int(np.argmax(got[-1].astype(np.float32)))
        if ref:
            refl.append(ref.decode(emb[ids[S + t]]))
    engine.shutdown()
    return got, refl


def _check(got, refl, min_cos):
    for step, (g, r) in enumerate(zip(got, refl)):
        gf, rf = g.astype(np.float32), r.astype(np.float32)
        assert np.isfinite(gf).all()
        c = cosine(gf, rf)
        top = np.sort(rf)[-2:]
        margin = float(top[1] - top[0])
        assert c >= min_cos, f"step {step}: cos {c:.6f}"
        assert int(np.argmax(gf)) == int(np.argmax(rf)), f"step {step}: top-1 differs (ref margin {margin:.3g})"


def test_small_model_prefill_and_decode(engine):
    got, refl = _run(engine, SMALL, S=40, n_dec=6, seed=3)
    _check(got, refl, 0.9999)


def test_config4_layer_prefill_then_decode(engine):
    """BASELINE config 4 at its stated size: one 0.8B-class layer (hidden 1024, 16Q/8KV hd128,
    FFN 3072, vocab 151936), a 512-token prefill then 128 decode steps, teacher forced
    (engine and oracle consume the same ids), every step's logits against the oracle."""
    got, refl = _run(engine, CONFIG_08B_LAYER, S=512, n_dec=128, seed=5, max_pos=1024)
    _check(got, refl, 0.9999)


def test_decode_graph_replay_matches_direct(engine):
    """Decode steps replayed from the engine's HIP graph give the same bits as direct
    launches: every step's logits and token, with the host's input upload, output copy
    and temp read-back between replays."""
    prev = engine.set_graphs(False)
    try:
        c0, r0 = engine.graph_stats()
        direct, _ = _run(engine, SMALL, S=24, n_dec=10, seed=7, with_ref=False)
        assert engine.graph_stats() == (c0, r0)
        engine.set_graphs(True)
        graphed, _ = _run(engine, SMALL, S=24, n_dec=10, seed=7, with_ref=False)
        c1, r1 = engine.graph_stats()
    finally:
        engine.set_graphs(prev)
    assert c1 - c0 >= 1 and r1 - r0 >= 6, (c1 - c0, r1 - r0)
    for step, (a, b) in enumerate(zip(direct, graphed)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {step}"


def test_persistent_server_decode_matches_engine(engine, tmp_path):
    """Decode steps served by gehtp_persistent (a separate process holding the blob,
    its weights and the KV states) give the same logits bits as the same blob run in
    this process, and its token is the first maximum of those logits."""
    from gehtp_amd.persistent import SERVER, PersistentRuntime
    if not SERVER.exists():
        pytest.skip("server not built")
    cfg, steps = SMALL, 5
    w = Weights(cfg, seed=11)
    dec, td = emit_decode(cfg, w, 64)
    blob = tmp_path / "decode.wtop"
    blob.write_bytes(dec)
    (tmp_path / "decode.weights.bin").write_bytes(w.image.tobytes())
    emb = w.embed()
    ids = np.random.default_rng(12).integers(0, cfg.vocab, steps)
    bodies = [np.ascontiguousarray(emb[i]).tobytes() for i in ids]

    rt = PersistentRuntime(tmp_path / "persist", timeout=60.0)
    rt.start_server(blob, out_temp=td["logits"], in_bytes=len(bodies[0]), weights_size=w.image.nbytes)
    served = []
    try:
        for b in bodies:
            tok, resp, out = rt.run(b, want_out=True)
            served.append((tok, np.frombuffer(out, np.float16).copy()))
            assert resp["steps"] == len(served)
        rt.reset()                                   # fresh KV: step 0 again
        tok0, _, out0 = rt.run(bodies[0], want_out=True)
    finally:
        assert rt.stop_server() == 0

    engine.shutdown()
    engine.set_ext_weights(w.image.ctypes.data)
    engine.state_reset()
    pd = engine.parse(dec)
    for step, (b, (tok, logits)) in enumerate(zip(bodies, served)):
        engine.run_io(pd, b, td["logits"])
        mine = np.frombuffer(engine.temp(td["logits"]), np.float16)
        assert np.array_equal(mine.view(np.uint16), logits.view(np.uint16)), f"step {step}"
        assert tok == int(np.argmax(logits.astype(np.float32)))
    assert tok0 == served[0][0] and np.array_equal(np.frombuffer(out0, np.uint16), served[0][1].view(np.uint16))
    engine.shutdown()


@pytest.mark.parametrize("graphs", [True, False], ids=["graphs", "direct"])
def test_run_steps_matches_host_loop(engine, graphs):
    """wt_exec_run_steps with the token-id decode blob (embedding row gathered in-graph,
    each step's ARGMAX output fed back on the device) gives the tokens of the host loop
    that feeds wt_exec_run_io the embedding row of the previous token, step for step, and
    the same last-step logits bit for bit; the ring positions advance the same way."""
    cfg, S, n, max_pos = SMALL, 24, 40, 96
    w = Weights(cfg, seed=71)
    emb = w.embed()
    prev = engine.set_graphs(graphs)
    try:
        engine.shutdown()
        engine.set_ext_weights(w.image.ctypes.data)
        pre, tp = emit_prefill(cfg, w, S, max_pos)
        dec, td = emit_decode(cfg, w, max_pos)
        dect, tdt = emit_decode(cfg, w, max_pos, token_input=True)
        pp, pd, pt = engine.parse(pre), engine.parse(dec), engine.parse(dect)
        x_prompt = np.ascontiguousarray(emb[np.random.default_rng(72).integers(0, cfg.vocab, S)]).tobytes()

        engine.state_reset()
        out, _ = engine.run_io(pp, x_prompt, tp["tok"])
        tok = int(np.frombuffer(out, np.int32)[0])
        first = tok
        loop = []
        for _ in range(n):
            out, _ = engine.run_io(pd, emb[tok].tobytes(), td["tok"])
            tok = int(np.frombuffer(out, np.int32)[0])
            loop.append(tok)
        last_loop = np.frombuffer(engine.temp(td["logits"]), np.float16)[:cfg.vocab].copy()

        engine.state_reset()
        engine.run_io(pp, x_prompt, tp["tok"])
        c0, r0 = engine.graph_stats()
        chained = np.frombuffer(engine.run_steps(pt, n, np.int32(first).tobytes(), tdt["tok"]), np.int32)
        c1, r1 = engine.graph_stats()
        last_chained = np.frombuffer(engine.temp(tdt["logits"]), np.float16)[:cfg.vocab].copy()
        engine.shutdown()
    finally:
        engine.set_graphs(prev)
    assert chained.tolist() == loop
    assert np.array_equal(last_chained.view(np.uint16), last_loop.view(np.uint16))
    if graphs:
        assert r1 - r0 >= n - 4, (c1 - c0, r1 - r0)


def test_run_steps_errors(engine):
    """wt_exec_run_steps refuses an output larger than its 64 MiB limit before running
    anything, and stops with an error when out_temp does not hold as many bytes as the
    input slot (here the logits temp of the token-id decode blob)."""
    cfg, max_pos = SMALL, 64
    w = Weights(cfg, seed=73)
    engine.shutdown()
    engine.set_ext_weights(w.image.ctypes.data)
    dect, tdt = emit_decode(cfg, w, max_pos, token_input=True)
    pt = engine.parse(dect)
    engine.state_reset()
    first = np.int32(5).tobytes()
    with pytest.raises(ValueError, match="64 MiB"):   # the Python mirror checks first
        engine.run_steps(pt, 20_000_000, first, tdt["tok"])
    # the library's own check, called directly: it refuses before writing any output
    import ctypes as C
    err, m, obuf = C.create_string_buffer(256), C.c_uint32(0), C.create_string_buffer(16)
    rc = engine.lib.wt_exec_run_steps(C.byref(pt.blob), 20_000_000, C.c_char_p(first), obuf, tdt["tok"],
                                      C.byref(m), err, 256)
    assert rc != 0 and b"output limit" in err.value, (rc, err.value)
    with pytest.raises(RuntimeError, match="output temp"):
        engine.run_steps(pt, 2, first, tdt["logits"])
    ids = np.frombuffer(engine.run_steps(pt, 3, first, tdt["tok"]), np.int32)
    assert ids.shape == (3,) and (ids >= 0).all() and (ids < cfg.vocab).all()
    engine.shutdown()


def _run_plain_vs_planned(engine, cfg, S, n_dec, seed, max_pos, **plan):
    """Prompt + teacher-forced decode steps through this build's blobs, plain and with
    `plan` (recycle / tempoff); returns the logits rows of both."""
    w = Weights(cfg, seed=seed)
    ids = np.random.default_rng(seed + 1).integers(0, cfg.vocab, S + n_dec)
    emb = w.embed()
    out = []
    for kw in ({}, plan):
        engine.shutdown()
        engine.set_ext_weights(w.image.ctypes.data)
        pre, tp = emit_prefill(cfg, w, S, max_pos, **kw)
        dec, td = emit_decode(cfg, w, max_pos, **kw)
        pp, pd = engine.parse(pre), engine.parse(dec)
        engine.state_reset()
        engine.run_io(pp, np.ascontiguousarray(emb[ids[:S]]).tobytes(), tp["tok"])
        rows = [np.frombuffer(engine.temp(tp["logits"]), np.float16)[:cfg.vocab].copy()]
        for t in range(n_dec):
            engine.run_io(pd, emb[ids[S + t]].tobytes(), td["tok"])
            rows.append(np.frombuffer(engine.temp(td["logits"]), np.float16)[:cfg.vocab].copy())
        # the prefill blob again after the decode blob (with plans: back to its own plan)
        engine.state_reset()
        engine.run_io(pp, np.ascontiguousarray(emb[ids[:S]]).tobytes(), tp["tok"])
        again = np.frombuffer(engine.temp(tp["logits"]), np.float16)[:cfg.vocab]
        assert np.array_equal(again.view(np.uint16), rows[0].view(np.uint16)), "prefill after decode"
        engine.shutdown()
        out.append(rows)
    return out


@pytest.mark.parametrize("plan", [{"tempoff": True}, {"recycle": True, "tempoff": True}],
                         ids=["tempoff", "recycled-tempoff"])
@pytest.mark.parametrize("cfg,S,n_dec,max_pos", [(SMALL, 40, 12, 96), (CONFIG_08B_LAYER, 512, 24, 600)],
                         ids=["small-2layer", "config4"])
def test_static_temp_plan_gives_the_same_bits(engine, cfg, S, n_dec, max_pos, plan):
    """The model's prefill and decode blobs with a TEMPOFF static plan (temps whose values
    never meet share bytes: the SwiGLU activation over the attention tensors), with and
    without recycled temp ids, give the bits of the same blobs with bump-allocated temps,
    at every step (graph replay on, as by default). Each blob runs on its own plan: the
    decode blob's replaces the prefill blob's, and the prefill blob run again afterwards
    gets its own back."""
    plain, planned = _run_plain_vs_planned(engine, cfg, S, n_dec, 61, max_pos, **plan)
    for t, (a, b) in enumerate(zip(plain, planned)):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"step {t}"
