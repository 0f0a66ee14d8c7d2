"""Writes tests/golden/e2e_4b_seed0.npz: the CPU golden of BASELINE config 5 (run from the
repo root, in the build container; about 15 minutes on 8 cores).

The 4B-class Qwen3-style model (36 layers, hidden 2560, 32 Q / 8 KV heads at head_dim 128,
SwiGLU FFN 9728, vocab 151936 with the fp16 embedding as lm_head, all other linears
W4A16 group 64), random-initialised by gehtp_amd.qwen3.Weights(seed), runs through the
oracle's restatement of the reference runlist (oracle/qwen3_ref.py: every op the
reference's scalar arithmetic with f16 rounding at op boundaries, attention as the
batched-matmul / scale / mask / softmax / matmul chain): a prompt of 2048 seeded token
ids, then T greedy decode steps, each fed the oracle's own argmax (teacher forcing for
the engine under test, which consumes the same ids).

Saved per logits row (row 0 = the prompt's last token, row t = decode step t):
argmax, the top two values, the 64 largest logits (index, value), and every 8th logit
(for a cosine), plus the ids, the weight image's CRC32 (so a test can check it rebuilt
the same weights), and the shapes.

The order-only spread: the same model runs twice more with the oracle's other valid
fp32 summation orders (oracle.summation_order 1: 32-wide slices combined pairwise, the
decode GEMV's shape; 2: 16-deep slices added in sequence, the MFMA GEMM's K steps;
attention's P.V in 64-key chunks), with the same products and f16 rounding points,
teacher-forced on the same ids. For each row, `band` is the largest difference, over
both orders and the 64 golden leaders, between an alternative order's logit and the
golden's: how far a correct implementation's logits move with the summation order
alone. `alt_argmax` / `alt_top2` hold each order's own leader and two best values.

    python tests/golden/make_e2e_4b.py [--steps 32] [--threads 8]
"""
from __future__ import annotations

import argparse
import sys
import time
import zlib
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from gehtp_amd.qwen3 import CONFIG_4B, Weights  # noqa: E402
from oracle import oracle as o  # noqa: E402
from oracle.qwen3_ref import RefModel  # noqa: E402

OUT = Path(__file__).resolve().parent / "e2e_4b_seed0.npz"
STRIDE = 8
TOPK = 64


def image_crc(img: np.ndarray) -> int:
    crc = 0
    step = 1 << 26
    for o in range(0, img.size, step):
        crc = zlib.crc32(img[o:o + step], crc)
    return crc


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--orders", type=int, nargs="*", default=[1, 2])
    args = ap.parse_args()
    cfg, S, T = CONFIG_4B, args.prompt, args.steps
    t0 = time.time()
    w = Weights(cfg, seed=args.seed)
    crc = image_crc(w.image)
    print(f"weights {w.image.nbytes / 1e9:.2f} GB crc {crc:#010x} in {time.time() - t0:.0f}s", flush=True)
    ids = np.random.default_rng(args.seed + 1).integers(0, cfg.vocab, S).astype(np.int32)
    emb = w.embed()
    ref = RefModel(cfg, w, max_pos=S + T + 8, threads=args.threads)
    rows = []
    t0 = time.time()
    logits = ref.prefill(np.ascontiguousarray(emb[ids]))
    rows.append(logits)
    print(f"prefill {S} tokens in {time.time() - t0:.0f}s: argmax {int(np.argmax(logits))}", flush=True)
    dec_ids = []
    for t in range(T):
        nxt = int(np.argmax(rows[-1].astype(np.float32)))
        dec_ids.append(nxt)
        t1 = time.time()
        rows.append(ref.decode(emb[nxt]))
        print(f"decode {t}: fed {nxt}, argmax {int(np.argmax(rows[-1]))} ({time.time() - t1:.1f}s)", flush=True)
    L = np.stack(rows).astype(np.float32)
    order = np.argsort(-L, axis=1, kind="stable")[:, :TOPK]
    gold_top = np.take_along_axis(L, order, axis=1)
    alt_argmax, alt_top2, alt_dev = [], [], []
    for mode in args.orders:
        with o.summation_order(mode):
            ref = RefModel(cfg, w, max_pos=S + T + 8, threads=args.threads)
            t0 = time.time()
            alt = [ref.prefill(np.ascontiguousarray(emb[ids]))]
            for nxt in dec_ids:   # teacher forced on the golden's ids
                alt.append(ref.decode(emb[nxt]))
        A = np.stack(alt).astype(np.float32)
        alt_argmax.append(np.argmax(A, axis=1).astype(np.int32))
        alt_top2.append(-np.sort(-A, axis=1)[:, :2])
        dev = np.abs(np.take_along_axis(A, order, axis=1) - gold_top).max(axis=1)
        alt_dev.append(dev)
        print(f"order {mode}: {time.time() - t0:.0f}s, top-64 deviation per row max {dev.max():.4g} "
              f"median {float(np.median(dev)):.4g}, argmax differs at rows "
              f"{[int(r) for r in np.nonzero(alt_argmax[-1] != np.argmax(L, axis=1))[0]]}", flush=True)
    band = np.max(np.stack(alt_dev), axis=0).astype(np.float32) if alt_dev else np.zeros(len(rows), np.float32)
    np.savez_compressed(
        OUT, seed=args.seed, prompt=S, steps=T, vocab=cfg.vocab, image_crc=np.uint32(crc),
        prompt_ids=ids, decode_ids=np.array(dec_ids, np.int32),
        argmax=np.argmax(L, axis=1).astype(np.int32),
        top2=np.take_along_axis(L, order[:, :2], axis=1).astype(np.float32),
        top_idx=order.astype(np.int32), top_val=np.stack(rows)[np.arange(len(rows))[:, None], order],
        stride=STRIDE, logits_strided=np.stack(rows)[:, ::STRIDE],
        orders=np.array(args.orders, np.int32), band=band,
        alt_argmax=np.array(alt_argmax, np.int32).reshape(len(args.orders), len(rows)),
        alt_top2=np.array(alt_top2, np.float32).reshape(len(args.orders), len(rows), 2))
    print(f"wrote {OUT} ({OUT.stat().st_size / 1e6:.2f} MB)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
