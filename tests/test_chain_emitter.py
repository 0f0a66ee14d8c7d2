"""The chain-form runlist emitter (gehtp_amd.qwen3_chain) on the CPU: its blobs parse,
carry the reference chain's opcodes (and none of this build's fused ones), and the
decode step body is the reference runner's (scripts/persistent_runtime.py:43-62)."""
from __future__ import annotations

import collections

import numpy as np

from gehtp_amd import Engine
from gehtp_amd.qwen3 import Qwen3Config, Weights
from gehtp_amd.qwen3_chain import decode_input, emit_decode_chain, emit_prefill_chain, face_elems, rope_tables

SMALL = Qwen3Config(layers=2, hidden=512, heads=4, kv_heads=2, ffn=1024, vocab=3000)


def _hist(blob):
    pb = Engine().parse(blob)
    return collections.Counter(pb.blob.ops[i].opcode for i in range(pb.n_ops)), pb.n_ops


def test_decode_chain_opcodes():
    w = Weights(SMALL, seed=1)
    hist, n = _hist(emit_decode_chain(SMALL, w, 64)[0])
    L = SMALL.layers
    # per layer: 22, 23, 24 x 2, 13, 7; RoPE 15 x 2 + 11 + 14 per q and k; 40 x 6
    assert hist[22] == L and hist[23] == L and hist[24] == 2 * L + 1 and hist[13] == L and hist[7] == L
    assert hist[40] == 6 * L and hist[14] == 2 * L and hist[20] == 1 and hist[21] == 1
    assert hist[15] == 3 + 6 * L and hist[26] == 5 and hist[11] == 3 * L
    assert not ({41, 42, 43, 44, 45, 46, 47} & set(hist)), "the chain form uses no fused opcode"


def test_prefill_chain_opcodes():
    w = Weights(SMALL, seed=1)
    hist, _ = _hist(emit_prefill_chain(SMALL, w, 16)[0])
    L = SMALL.layers
    assert hist[27] == 4 * L and hist[26] == 4 + 2 * L and hist[24] == 2 * L + 1 and hist[13] == L
    assert 22 not in hist and 23 not in hist


def test_decode_input_face():
    P = 16
    body = decode_input(SMALL, 1234, 0, P)
    assert len(body) == face_elems(SMALL, P) * 2
    assert np.frombuffer(body[:4], np.int32)[0] == 1234
    f = np.frombuffer(body[4:], np.float16)
    cos, sin, mask = f[:128], f[128:256], f[256:]
    assert (cos == 1).all() and (sin == 0).all()                # position 0
    assert mask[0] == 0 and np.isneginf(mask[1:]).all()
    body = decode_input(SMALL, 7, 5, P)
    f = np.frombuffer(body[4:], np.float16)
    c, s = rope_tables(np.array([5]), 128, SMALL.theta)
    assert np.array_equal(f[:128], c[0]) and np.array_equal(f[128:256], s[0])
    assert np.array_equal(f[:64], f[64:128])                     # each half duplicated
    # pair 0 rotates by exactly the position (inv_freq 1)
    assert f[0] == np.float16(np.cos(5.0)) and f[128] == np.float16(np.sin(5.0))
    assert (f[256:256 + 6] == 0).all() and np.isneginf(f[256 + 6:]).all()
