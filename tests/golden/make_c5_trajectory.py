"""Writes tests/golden/c5_trajectory.json: the CPU oracle's losses over 200
training steps of the C5 char-nanoGPT (V=65, T=256, C=384, H=6, L=6, B=64;
AdamW lr 1e-3, betas (0.9, 0.99), eps 1e-8, weight decay 0.1; weights
randn * 0.02 from Philox call 0), the step of
examples/nanogpt_modular.ml:167-189.

The batches are windows of a learnable token stream (a fixed 97-token
phrase repeated, a tenth of the positions replaced by random tokens), so the
loss falls from ln(65) ~ 4.17 and a wrong gradient shows in the trajectory.
`batch(step)` builds them from numpy's PCG64 streams, which are the same on
every machine; the fixture also keeps a checksum of every batch so a test
can tell that it trains on the same tokens.

Run in the build container (8 cores, about 30 s per step):
    python tests/golden/make_c5_trajectory.py [steps] [checkpoint.npz]
Every 10 steps the oracle's parameters, moments and losses go to the
checkpoint (default /tmp/c5_trajectory_ckpt.npz), and a new run resumes
from it.
"""
from __future__ import annotations

import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "c5_trajectory.json"

C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)
CORPUS_SEED, CORPUS_LEN, PHRASE = 11, 1 << 20, 97


def corpus():
    rng = np.random.default_rng(CORPUS_SEED)
    phrase = rng.integers(0, C5["V"], PHRASE)
    data = np.resize(phrase, CORPUS_LEN)
    noise = rng.random(CORPUS_LEN) < 0.1
    data[noise] = rng.integers(0, C5["V"], int(noise.sum()))
    return data.astype(np.int32)


def batch(data, step):
    """Token and target ids of step `step` (1-based): B windows of T + 1
    tokens at starts drawn from PCG64(1000 + step)."""
    rng = np.random.default_rng(1000 + step)
    starts = rng.integers(0, len(data) - C5["T"] - 1, C5["B"])
    x = np.concatenate([data[s:s + C5["T"]] for s in starts]).astype(np.int32)
    y = np.concatenate([data[s + 1:s + C5["T"] + 1] for s in starts]).astype(np.int32)
    return x, y


def checksum(x, y):
    w = np.arange(1, x.size + 1, dtype=np.int64)
    return int((w * x).sum() + 3 * (w * y).sum())


def _save(path, g, losses, sums):
    arrs = {"losses": np.array(losses, np.float64), "sums": np.array(sums, np.int64)}
    for i in range(g.nparams):
        arrs[f"p{i}"] = g.param(i)
        arrs[f"m{i}"] = g.moment(i, 0)
        arrs[f"v{i}"] = g.moment(i, 1)
    tmp = Path(str(path) + ".tmp.npz")
    np.savez(tmp, **arrs)
    os.replace(tmp, path)


def _load(path, g):
    with np.load(path) as z:
        for i in range(g.nparams):
            g.set_param(i, z[f"p{i}"])
            g.set_moment(i, 0, z[f"m{i}"])
            g.set_moment(i, 1, z[f"v{i}"])
        return [float(v) for v in z["losses"]], [int(v) for v in z["sums"]]


def _write(losses, sums):
    OUT.write_text(json.dumps({
        "about": "CPU oracle (oracle/malus_oracle.c) losses of C5 training steps 1..n on the corpus "
                 "and batches of tests/golden/make_c5_trajectory.py; f32 values printed as Python floats",
        "config": C5, "optimizer": OPT, "init": "randn * 0.02, Philox call index 0",
        "corpus": {"seed": CORPUS_SEED, "length": CORPUS_LEN, "phrase": PHRASE, "noise": 0.1},
        "batch_seed": "PCG64(1000 + step)",
        "losses": losses, "batch_checksums": sums}, indent=1) + "\n")


def main(steps=200, ckpt="/tmp/c5_trajectory_ckpt.npz"):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O

    O.set_threads(os.cpu_count() or 1)
    data = corpus()
    g = O.Gpt(**C5, **OPT)
    losses, sums = ([], []) if not os.path.exists(ckpt) else _load(ckpt, g)
    t0 = time.time()
    for t in range(len(losses) + 1, steps + 1):
        x, y = batch(data, t)
        losses.append(float(g.step(x, y, t)))
        sums.append(checksum(x, y))
        print(f"step {t}: loss {losses[-1]:.6f} ({time.time() - t0:.0f} s)", flush=True)
        if t % 10 == 0 or t == steps:
            _save(ckpt, g, losses, sums)
            _write(losses, sums)


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 200, *sys.argv[2:3])
