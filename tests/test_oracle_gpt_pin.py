"""Pins the oracle's nanoGPT composition (or_gpt_loss_and_grads, or_gpt_step)
against an independent float64 restatement of the reference program.

The restatement below is written from examples/nanogpt_modular.ml:38-108
alone, with torch float64 tensors on the CPU and torch autograd for the
gradients; it shares no code with oracle/malus_oracle.c.  A composition
mistake in the oracle (head fold order, which tensor a residual adds, the
LN-weight index, mask orientation, the optimizer's expression) changes the
float64 loss or a gradient far beyond float32 rounding and fails here.
CPU only.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")

CFG = dict(V=11, T=8, C=16, H=4, L=2, B=2)


def _ln(x):
    """layernorm(x, axis=1): population variance, eps 1e-5, no affine
    (layernorm.ml:1-31; metal.rs:1486-1533)."""
    mu = x.mean(dim=1, keepdim=True)
    var = ((x - mu) ** 2).mean(dim=1, keepdim=True)
    return (x - mu) / torch.sqrt(var + 1e-5)


def _gelu(x):
    """tanh-approximation GELU with the constants of gelu.ml:5-14."""
    c0, c1 = 0.7978845608028654, 0.044715
    return 0.5 * x * (1.0 + torch.tanh(c0 * (x + c1 * x ** 3)))


def _forward(params, toks, tgts, cfg):
    """GPT.forward + cross_entropy (nanogpt_modular.ml:75-91, 38-68)."""
    V, T, C, H, L, B = (cfg[k] for k in ("V", "T", "C", "H", "L", "B"))
    hs = C // H
    n = B * T
    wte, wpe, ln_f, lm_head = params[8 * L: 8 * L + 4]
    pos = torch.arange(T).repeat(B)  # pos_buf[b*T+t] = t
    x = wte[toks] + wpe[pos]
    # causal_mask(T): 0 on and below the diagonal, -1e9 above (metal.rs:1600-1612)
    mask = torch.triu(torch.full((T, T), -1e9, dtype=torch.float64), diagonal=1)
    scale = 1.0 / math.sqrt(hs)
    for l in range(L):
        ln1_w, wq, wk, wv, wo, ln2_w, w1, w2 = params[8 * l: 8 * l + 8]
        xn1 = _ln(x) * ln1_w

        def heads(m):  # reshape(permute(reshape(m, B,T,H,hs), 0,2,1,3), B*H, T, hs)
            return m.reshape(B, T, H, hs).permute(0, 2, 1, 3).reshape(B * H, T, hs)

        q, k, v = heads(xn1 @ wq), heads(xn1 @ wk), heads(xn1 @ wv)
        scores = (q @ k.transpose(1, 2)) * scale + mask
        att = torch.softmax(scores, dim=2)
        out = (att @ v).reshape(B, H, T, hs).permute(0, 2, 1, 3).reshape(n, C)
        x2 = x + out @ wo
        xn2 = _ln(x2) * ln2_w
        x = x2 + _gelu(xn2 @ w1) @ w2
    logits = (_ln(x) * ln_f) @ lm_head
    # cross_entropy: mean over rows of -log(softmax(logits)[target]) (cross_entropy.ml:13-28)
    logp = torch.log_softmax(logits, dim=1)
    loss = -logp[torch.arange(n), tgts].mean()
    return loss, logits


def _adam_l2(p, g, m, v, t, lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1):
    """The reference 'adamw' (nanogpt_modular.ml:97-108): coupled L2 decay."""
    gg = g + wd * p
    m = b1 * m + (1.0 - b1) * gg
    v = b2 * v + (1.0 - b2) * gg * gg
    m_hat = m / (1.0 - b1 ** t)
    v_hat = v / (1.0 - b2 ** t)
    return p - lr * m_hat / (np.sqrt(v_hat) + eps), m, v


def _shapes(cfg):
    V, T, C, L = cfg["V"], cfg["T"], cfg["C"], cfg["L"]
    blk = [(C,), (C, C), (C, C), (C, C), (C, C), (C,), (C, 4 * C), (4 * C, C)]
    return blk * L + [(V, C), (T, C), (C,), (C, V)]


def _params64(og, cfg, perturb_ln=False):
    """The oracle's parameters as float64 leaves; optionally moves the LN
    weights off 1 (in the oracle too) so a wrong LN-weight index shows."""
    shapes = _shapes(cfg)
    out = []
    rng = np.random.default_rng(3)
    for i, s in enumerate(shapes):
        p = og.param(i)
        if perturb_ln and len(s) == 1:
            p = (1.0 + 0.3 * rng.standard_normal(p.size)).astype(np.float32)
            og.set_param(i, p)
        out.append(torch.tensor(p.astype(np.float64).reshape(s), requires_grad=True))
    return out


def _tokens(cfg, seed):
    n = cfg["B"] * cfg["T"]
    return O.rand_tokens(seed, n, cfg["V"]), O.rand_tokens(seed + n, n, cfg["V"])


@pytest.mark.parametrize("perturb_ln", [False, True], ids=["ln_ones", "ln_perturbed"])
def test_oracle_gpt_loss_logits_and_grads_match_float64_restatement(perturb_ln):
    og = O.Gpt(**CFG)
    ps = _params64(og, CFG, perturb_ln)
    x, y = _tokens(CFG, 11)
    loss64, logits64 = _forward(ps, torch.tensor(x, dtype=torch.long), torch.tensor(y, dtype=torch.long), CFG)
    loss64.backward()
    loss32, logits32 = og.loss_and_grads(x, y, want_logits=True)
    lw = float(loss64.detach())
    assert abs(float(loss32) - lw) <= 1e-5 * abs(lw), (float(loss32), lw)
    lg = logits64.detach().numpy()
    assert np.max(np.abs(logits32 - lg)) <= 1e-5 * np.max(np.abs(lg))
    for i, p in enumerate(ps):
        want = p.grad.numpy().ravel()
        got = og.grad(i).astype(np.float64)
        err = np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30)
        assert err <= 1e-4, f"param {i}: normwise gradient error {err:.2e}"


def test_oracle_gpt_initial_loss_is_near_log_vocab():
    # N(0, 0.02) weights make the logits nearly uniform: loss ~ ln(V)
    og = O.Gpt(**CFG)
    x, y = _tokens(CFG, 5)
    loss = float(og.loss_and_grads(x, y))
    assert abs(loss - math.log(CFG["V"])) < 0.05, loss


def test_oracle_gpt_three_adam_steps_match_float64_restatement():
    og = O.Gpt(**CFG)
    ps = [p.detach().numpy().copy() for p in _params64(og, CFG)]
    p0 = [p.copy() for p in ps]
    ms = [np.zeros_like(p) for p in ps]
    vs = [np.zeros_like(p) for p in ps]
    for t in (1, 2, 3):
        x, y = _tokens(CFG, 100 * t)
        leaves = [torch.tensor(p, requires_grad=True) for p in ps]
        loss64, _ = _forward(leaves, torch.tensor(x, dtype=torch.long), torch.tensor(y, dtype=torch.long), CFG)
        loss64.backward()
        loss32 = float(og.step(x, y, t))
        lw = float(loss64.detach())
        assert abs(loss32 - lw) <= 1e-5 * abs(lw), (t, loss32, lw)
        for i in range(len(ps)):
            ps[i], ms[i], vs[i] = _adam_l2(ps[i], leaves[i].grad.numpy(), ms[i], vs[i], t)
    for i in range(len(ps)):
        want = (ps[i] - p0[i]).ravel()
        got = og.param(i).astype(np.float64) - p0[i].ravel()
        # the updates are ~lr per element; compare them normwise
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        assert err <= 1e-3, f"param {i}: update error {err:.2e} after 3 steps"
