"""Writes the CPU oracle's losses over 200 training steps of the C5
char-nanoGPT (V=65, T=256, C=384, H=6, L=6, B=64; AdamW lr 1e-3, betas
(0.9, 0.99), eps 1e-8, weight decay 0.1; weights randn * 0.02 from Philox
call 0), the step of examples/nanogpt_modular.ml:167-189, on two kinds of
batches:

  iid     tests/golden/c5_trajectory_iid.json: the configuration's own data,
          token and target ids i.i.d. uniform in [0, 65), drawn by the
          `rand_int` builtin with call indices `iid_calls(step)` (the ids
          malus_rand_tokens_device draws on the device);
  corpus  tests/golden/c5_trajectory.json: windows of a learnable token
          stream (a fixed 97-token phrase repeated, a tenth of the positions
          replaced by random tokens), so the loss falls from ln(65) ~ 4.17;
          `batch(step)` builds them from numpy's PCG64 streams, which are the
          same on every machine.  At this learning rate the run learns the
          phrase through a sharp transition (steps ~20-40), plateaus near
          1.8 and turns unstable from step ~85; in the transition and after
          it, runs that differ in the last bit part ways (the tests compare
          the plateau, not every step).  The committed fixture holds 150
          steps.

Each fixture keeps a checksum of every batch so a test can tell that it
trains on the same tokens.

Run in the build container (8 cores, about 15-30 s per step):
    python tests/golden/make_c5_trajectory.py {iid|corpus} [steps] [checkpoint.npz]
Every 10 steps the oracle's parameters, moments and losses go to the
checkpoint (default /tmp/c5_trajectory_<kind>_ckpt.npz), and a new run
resumes from it.
"""
from __future__ import annotations

import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
HERE = Path(__file__).resolve().parent
OUT = {"corpus": HERE / "c5_trajectory.json", "iid": HERE / "c5_trajectory_iid.json"}

C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)
CORPUS_SEED, CORPUS_LEN, PHRASE = 11, 1 << 20, 97
N_TOK = C5["B"] * C5["T"]


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


def iid_calls(step):
    """The `rand_int` call indices of step `step`'s token ids (x[i] with
    cx + i, y[i] with cy + i)."""
    cx = (3 << 32) + 2 * N_TOK * step
    return cx, cx + N_TOK


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


def _write(kind, losses, sums):
    data = ({"corpus": {"seed": CORPUS_SEED, "length": CORPUS_LEN, "phrase": PHRASE, "noise": 0.1},
             "batch_seed": "PCG64(1000 + step)"} if kind == "corpus" else
            {"ids": "rand_int(65) per token, call indices iid_calls(step)"})
    OUT[kind].write_text(json.dumps({
        "about": f"CPU oracle (oracle/malus_oracle.c) losses of C5 training steps 1..n on the {kind} batches of "
                 "tests/golden/make_c5_trajectory.py; f32 values printed as Python floats",
        "config": C5, "optimizer": OPT, "init": "randn * 0.02, Philox call index 0", **data,
        "losses": losses, "batch_checksums": sums}, indent=1) + "\n")


def main(kind, steps=200, ckpt=None):
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O

    ckpt = ckpt or f"/tmp/c5_trajectory_{kind}_ckpt.npz"
    O.set_threads(os.cpu_count() or 1)
    data = corpus() if kind == "corpus" else None
    g = O.Gpt(**C5, **OPT)
    losses, sums = ([], []) if not os.path.exists(ckpt) else _load(ckpt, g)
    t0 = time.time()
    for t in range(len(losses) + 1, steps + 1):
        if kind == "corpus":
            x, y = batch(data, t)
        else:
            cx, cy = iid_calls(t)
            x, y = O.rand_tokens(cx, N_TOK, C5["V"]), O.rand_tokens(cy, N_TOK, C5["V"])
        losses.append(float(g.step(x, y, t)))
        sums.append(checksum(x, y))
        print(f"step {t}: loss {losses[-1]:.6f} ({time.time() - t0:.0f} s)", flush=True)
        if t % 10 == 0 or t == steps:
            _save(ckpt, g, losses, sums)
            _write(kind, losses, sums)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 200, *sys.argv[3:4])
