"""The device-side data path and checkpoints: randn generated on the device
against the host stream (tensor_randn, metal.rs:1720-1740) and the oracle;
batches built on the device against the host loop of
nanogpt_modular.ml:170-177 (rand_int per sequence, then the windows); the
SafeTensors checkpoint read back by the `safetensors` package and resumed
bit for bit."""
import ctypes as C

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_bitexact, ulp_dist

pytestmark = pytest.mark.gpu

OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


@pytest.mark.parametrize("shape", [(1001,), (257, 384), (2,), (1,)])
def test_randn_device_is_the_host_stream(rt, shape):
    L = rt.L
    L.malus_rng_set_counter(40)
    hh = L.tensor_randn(M.sizes(shape), len(shape))
    after_host = L.malus_rng_get_counter()
    L.malus_rng_set_counter(40)
    hd = L.malus_randn_device(M.sizes(shape), len(shape))
    assert L.malus_rng_get_counter() == after_host == 41
    host, dev = rt.numpy(hh), rt.numpy(hd)
    # the same Philox words and the same f64 Box-Muller: equal, but for a
    # double-rounding tie at most (the device's f64 log/sin/cos are not the
    # host libm's, so a last-bit difference of a double can cross an f32
    # rounding boundary, with probability ~1e-9 per value)
    d = ulp_dist(dev, host)
    assert d.max() <= 1 and np.count_nonzero(d) <= max(1, dev.size // 100000)
    assert_bitexact(host, O.randn(40, shape).reshape(shape), "host randn vs oracle")
    rt.free(hh, hd)


def test_batch_windows_are_the_host_loop(rt):
    L = rt.L
    rng = np.random.default_rng(5)
    data = rng.integers(0, 65, 5000).astype(np.int32)
    hdata = rt.tensor(data)
    B, T = 16, 64
    L.malus_rng_set_counter(1000)
    starts_host = [L.malus_rand_int(len(data) - T - 1) for _ in range(B)]  # nanogpt_modular.ml:172
    x_want = np.concatenate([data[s:s + T] for s in starts_host])
    y_want = np.concatenate([data[s + 1:s + T + 1] for s in starts_host])
    # the oracle's Philox restatement gives the same starts
    assert starts_host == [O.philox([1, 0, 0, 0], [1000 + b, 0])[0] % (len(data) - T - 1) for b in range(B)]
    L.malus_rng_set_counter(1000)
    hx, hy = C.c_int64(), C.c_int64()
    starts = (C.c_int32 * B)()
    L.malus_batch_windows(hdata, B, T, C.byref(hx), C.byref(hy), starts)
    assert L.malus_rng_get_counter() == 1000 + B
    assert list(starts) == starts_host
    np.testing.assert_array_equal(rt.numpy(hx.value), x_want)
    np.testing.assert_array_equal(rt.numpy(hy.value), y_want)
    rt.free(hdata, hx.value, hy.value)


@pytest.mark.parametrize("call,n,vocab", [(0, 16384, 65), ((1 << 32) - 100, 1000, 65), (7, 1, 1), (123, 777, 1024),
                                         ((5 << 40) + 3, 70000, 50257)])
def test_rand_tokens_device_is_the_host_draw(rt, call, n, vocab):
    # the device draw equals the host builtin's loop (rand_int per token with
    # call index call + i), key words crossing 2^32 included
    h = rt.L.malus_rand_tokens_device(call, n, vocab)
    assert h, rt.last_error()
    got = rt.numpy(h)
    rt.free(h)
    assert got.dtype == np.int32
    assert_bitexact(got, O.rand_tokens(call, n, vocab), f"rand_tokens call {call} n {n} vocab {vocab}")


def test_batch_windows_rejects_short_data(rt):
    hdata = rt.tensor(np.arange(10, dtype=np.int32))
    hx, hy = C.c_int64(), C.c_int64()
    rt.L.malus_set_abort_on_error(0)
    try:
        rt.L.malus_batch_windows(hdata, 2, 9, C.byref(hx), C.byref(hy), None)
        assert "cannot hold a window" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(hdata)


def _gpt(rt, cfg, counter):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(counter)
    return rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"], OPT["b1"],
                                 OPT["b2"], OPT["eps"], OPT["wd"])


def _step(rt, g, x, y, t):
    hx, hy = rt.tensor(x), rt.tensor(y)
    hl = rt.L.malus_gpt_step(g, hx, hy, t)
    loss = rt.numpy(hl)[0]
    rt.free(hl, hx, hy)
    return loss


def test_checkpoint_resume_is_bit_identical_and_readable(rt, tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    from safetensors import safe_open

    cfg = dict(V=65, T=64, C=128, H=4, L=2, B=4)
    n = cfg["B"] * cfg["T"]
    batches = [(O.rand_tokens(70 + 2 * k, n, cfg["V"]), O.rand_tokens(71 + 2 * k, n, cfg["V"])) for k in range(5)]
    path = str(tmp_path / "gpt.safetensors")
    g = _gpt(rt, cfg, 0)
    for k in range(3):
        _step(rt, g, *batches[k], k + 1)
    assert rt.L.malus_gpt_save(g, path.encode(), 3) == 0
    want = [_step(rt, g, *batches[k], k + 1) for k in (3, 4)]
    params_want = [rt.numpy(rt.L.malus_gpt_param(g, i)) for i in range(rt.L.malus_gpt_nparams(g))]
    rt.L.malus_gpt_free(g)

    # the file as the safetensors package reads it
    tensors = st.load_file(path)
    assert len(tensors) == 3 * (8 * cfg["L"] + 4)
    assert tensors["blocks.1.w1"].shape == (cfg["C"], 4 * cfg["C"]) and tensors["wte"].dtype == np.float32
    with safe_open(path, framework="numpy") as f:
        assert f.metadata()["step"] == "3"

    # a model with another initialization resumes from the file
    g2 = _gpt(rt, cfg, 999)
    assert rt.L.malus_gpt_load(g2, path.encode()) == 3
    for i in range(rt.L.malus_gpt_nparams(g2)):
        name = (f"blocks.{i // 8}." + ["ln1_w", "wq", "wk", "wv", "wo", "ln2_w", "w1", "w2"][i % 8]
                if i < 8 * cfg["L"] else ["wte", "wpe", "ln_f", "lm_head"][i - 8 * cfg["L"]])
        np.testing.assert_array_equal(rt.numpy(rt.L.malus_gpt_param(g2, i)), tensors[name])
        np.testing.assert_array_equal(rt.numpy(rt.L.malus_gpt_moment(g2, i, 1)), tensors["adam_v." + name])
    got = [_step(rt, g2, *batches[k], k + 1) for k in (3, 4)]
    assert got == want
    for i, p in enumerate(params_want):
        np.testing.assert_array_equal(rt.numpy(rt.L.malus_gpt_param(g2, i)), p)
    # a mismatched model is refused
    bad = dict(cfg, C=64)
    g3 = _gpt(rt, bad, 0)
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.malus_gpt_load(g3, path.encode()) == -1
        assert "shape mismatching" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.L.malus_gpt_free(g2)
    rt.L.malus_gpt_free(g3)
    rt.L.tape_reset()


def test_checkpoint_with_malformed_offsets_is_refused(rt, tmp_path):
    import json
    import struct

    cfg = dict(V=65, T=16, C=32, H=4, L=1, B=2)
    path = tmp_path / "gpt.safetensors"
    g = _gpt(rt, cfg, 0)
    assert rt.L.malus_gpt_save(g, str(path).encode(), 1) == 0
    raw = path.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr, data = json.loads(raw[8:8 + n]), raw[8 + n:]
    before = [rt.numpy(rt.L.malus_gpt_param(g, i)) for i in range(rt.L.malus_gpt_nparams(g))]

    def write(h):
        b = json.dumps(h).encode()
        p = tmp_path / "bad.safetensors"
        p.write_bytes(struct.pack("<Q", len(b)) + b + data)
        return str(p).encode()

    wq, wk = hdr["blocks.0.wq"]["data_offsets"], hdr["blocks.0.wk"]["data_offsets"]
    cases = []
    h = json.loads(json.dumps(hdr))
    h["blocks.0.wq"]["data_offsets"] = [-8, wq[1] - wq[0] - 8]  # header bytes as data
    cases.append((h, "bad data offsets"))
    h = json.loads(json.dumps(hdr))
    h["blocks.0.wq"]["data_offsets"] = list(wk)  # two tensors on the same bytes
    cases.append((h, "overlap"))
    h = json.loads(json.dumps(hdr))
    h["blocks.0.wq"]["data_offsets"] = [len(data) - 4, len(data) - 4 + wq[1] - wq[0]]  # past the end
    cases.append((h, "bad data offsets"))
    h = json.loads(json.dumps(hdr))
    h["blocks.0.wq"]["data_offsets"] = ["0", str(wq[1] - wq[0])]  # not numbers
    cases.append((h, "data offsets"))
    rt.L.malus_set_abort_on_error(0)
    try:
        for h, msg in cases:
            assert rt.L.malus_gpt_load(g, write(h)) == -1
            assert msg in rt.last_error(), rt.last_error()
            rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    # nothing was read into the model
    for i, p in enumerate(before):
        np.testing.assert_array_equal(rt.numpy(rt.L.malus_gpt_param(g, i)), p)
    assert rt.L.malus_gpt_load(g, write(hdr)) == 1
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()
