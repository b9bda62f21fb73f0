"""Headline benchmark: warm-median ms/step of the Karpathy char-nanoGPT f32
training step on one MI355X.

A step = token upload (the `freeze` of buffer.rs:39-50) -> zero_grad ->
forward -> cross_entropy -> backward -> "AdamW" (examples/nanogpt_modular.ml:
167-189) through libmalus_hip's C ABI, with a device flush inside the timed
step (docs/adr/0038-benchmark-methodology.md).  Token batches are synthetic
(int32 i.i.d. uniform in [0, 65) from a fixed seed), built on the host before
timing and uploaded inside each timed step.  Prints ONE JSON line.

--config c4 runs the toy char-nanoGPT the same
way; --config c1 runs the XOR MLP's 10,000 steps.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CONFIGS = {
    "c5": dict(V=65, T=256, C=384, H=6, L=6, B=64),
    "c4": dict(V=65, T=64, C=128, H=4, L=4, B=32),
}
CFG = CONFIGS["c5"]
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)
METRIC = "warm-median ms/step, char-nanoGPT f32 train step; HBM GB/s & MFMA % of peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_BF16_MFMA_TFLOPS = 2500.0  # dense bf16 MFMA (no sparsity)
PEAK_HBM_GBS = 8000.0
ATTN_MODES = {"auto": 0, "flash": 1, "rows": 2, "composed": 3}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemm_flops_per_step(cfg) -> float:
    """Algorithmic GEMM FLOPs of one step: forward plus both VJP GEMMs."""
    B, T, Cn, H, L, V = cfg["B"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["V"]
    N, hs = B * T, Cn // H
    fwd_layer = 2 * N * Cn * Cn * 4 + 2 * N * Cn * 4 * Cn * 2 + 2 * (B * H) * T * T * hs * 2
    fwd = L * fwd_layer + 2 * N * Cn * V
    return 3.0 * fwd


def gemm_bytes_per_step(cfg) -> float:
    """Algorithmic HBM bytes of the step's GEMM launches (the k_sgemm class):
    each launch reads both operands and its epilogue operand once and writes
    its outputs once (4 bytes per element).  Every attention product (Q K^T,
    P @ V, dP = dO V^T, dQ = dS K, dK = dS^T Q and dV = P^T dO) runs inside
    the fused attention kernels, so none is counted here."""
    B, T, Cn, H, L, V = cfg["B"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["V"]
    N, F = B * T, 4 * cfg["C"]

    def one(m, n, k, batch=1):  # one GEMM launch
        return 4.0 * batch * (m * k + k * n + m * n)

    def mm(m, n, k, batch=1):  # a forward GEMM and its two VJP GEMMs (dA: m x k, dB: k x n)
        return 3 * one(m, n, k, batch)

    # epilogue operands: the GELU epilogue writes gelu(h) beside h and the
    # GELU VJP epilogue reads h; the two residual adds read their addend
    epi = 4.0 * (2 * N * F + 2 * N * Cn)
    layer = 4 * mm(N, Cn, Cn) + mm(N, F, Cn) + mm(N, Cn, F) + epi
    return L * layer + mm(N, V, Cn)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c5_gemm_hbm_traffic.txt")


def measured_traffic():
    """HBM bytes per step of all GEMM launches, as measured by the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs recorded in profiles/ (None if absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("gemm_hbm_bytes_per_step:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration(rt, sizes):
    """A plain copy of known size for counter calibration: out = x * 1.0 over
    2^26 f32 (256 MiB read, 256 MiB written), three launches."""
    L = rt.L
    x = L.tensor_alloc_ones_gpu(sizes((1 << 26,)), 1)
    for _ in range(3):
        y = L.malus_std_scalar_op(2, x, 1.0, 1)
        L.gpu_barrier()
        rt.free(y)
    rt.free(x)
    log("copy calibration: 3 x k_binary_scalar<MUL> over 2^26 f32 (268435456 B read + 268435456 B written each)")


def kernel_suite(rt, M, reps: int):
    """C2 (elementwise, 2^26 f32) and C3 (row ops on [65536, 1024]) kernels
    through the C ABI, each timed over `reps` launches between device
    flushes; bandwidth = algorithmic bytes / time (
    configs[2]).  Returns a list of rows; prints a table to stderr."""
    import numpy as np

    L = rt.L
    rng = np.random.default_rng(99)
    rows = []

    def timed(name, bytes_per_call, fn, shape):
        for _ in range(3):
            L.tensor_free(fn())
        L.gpu_barrier()
        t0 = time.perf_counter()
        for _ in range(reps):
            L.tensor_free(fn())
        L.gpu_barrier()
        dt = (time.perf_counter() - t0) / reps
        gbs = bytes_per_call / dt / 1e9
        rows.append({"op": name, "shape": shape, "us": round(dt * 1e6, 1), "GB/s": round(gbs, 1),
                     "frac_hbm": round(gbs / PEAK_HBM_GBS, 3), "bytes": int(bytes_per_call)})
        log(f"  {name:28s} {shape:14s} {dt * 1e6:8.1f} us  {gbs:7.1f} GB/s  {gbs / PEAK_HBM_GBS:5.1%} of HBM")

    # C2: z = a*b + 0.5*c - relu(a); r = A + bias, and the VJPs
    n = 1 << 26
    R, Cc = 8192, 8192
    a, b, c = (rt.tensor(rng.uniform(-1, 1, (R, Cc)).astype(np.float32)) for _ in range(3))
    bias = rt.tensor(rng.uniform(-1, 1, (1, Cc)).astype(np.float32))
    dz = L.tensor_alloc_ones_gpu(M.sizes((R, Cc)), 2)
    t1 = L.malus_std_broadcast_fwd(M.MUL, a, b)
    t2 = L.malus_std_scalar_op(M.MUL, c, 0.5, 0)
    t3 = L.malus_std_broadcast_fwd(M.ADD, t1, t2)
    t4 = L.malus_std_unary(M.RELU, a)
    log("C2 elementwise, [8192, 8192] f32:")
    timed("a * b", 12 * n, lambda: L.malus_std_broadcast_fwd(M.MUL, a, b), "8192x8192")
    timed("0.5 * c (scalar)", 8 * n, lambda: L.malus_std_scalar_op(M.MUL, c, 0.5, 0), "8192x8192")
    timed("t1 + t2", 12 * n, lambda: L.malus_std_broadcast_fwd(M.ADD, t1, t2), "8192x8192")
    timed("relu(a)", 8 * n, lambda: L.malus_std_unary(M.RELU, a), "8192x8192")
    timed("t3 - t4", 12 * n, lambda: L.malus_std_broadcast_fwd(M.SUB, t3, t4), "8192x8192")
    timed("A + bias (row broadcast)", 8 * n + 4 * Cc, lambda: L.malus_std_broadcast_fwd(M.ADD, a, bias), "8192x8192")
    timed("relu VJP", 12 * n, lambda: L.malus_std_relu_bwd(a, dz), "8192x8192")
    timed("mul VJP (dz * b)", 12 * n, lambda: L.malus_std_mul_bwd_a(dz, a, b), "8192x8192")
    timed("neg VJP (-dz)", 8 * n, lambda: L.malus_std_scale_fwd(dz, -1.0), "8192x8192")
    timed("bias VJP (sum over rows)", 4 * n + 4 * Cc, lambda: L.malus_std_sum_to_shape_bwd(dz, bias), "8192x8192")
    rt.free(a, b, c, bias, dz, t1, t2, t3, t4)

    # C3: row ops on [65536, 1024]
    Rr, V = 65536, 1024
    n = Rr * V
    x = rt.tensor(rng.standard_normal((Rr, V)).astype(np.float32))
    dout = rt.tensor(rng.standard_normal((Rr, V)).astype(np.float32))
    logits = rt.tensor((2.0 * rng.standard_normal((Rr, V))).astype(np.float32))
    tg = rt.tensor(rng.integers(0, V, Rr).astype(np.int32))
    sm = L.malus_std_softmax_fwd(x, 1)
    var = C.c_int64()
    ln = L.malus_std_layernorm_fwd(x, 1, C.byref(var))
    probs = C.c_int64()
    loss = L.malus_std_cross_entropy_fwd(logits, tg, C.byref(probs))
    one = L.tensor_alloc_ones_gpu(M.sizes((1,)), 1)
    log("C3 row ops, [65536, 1024] f32:")
    timed("softmax", 8 * n, lambda: L.malus_std_softmax_fwd(x, 1), "65536x1024")
    timed("softmax VJP", 12 * n, lambda: L.malus_std_softmax_bwd(sm, dout, 1), "65536x1024")

    def ln_fwd():
        v = C.c_int64()
        y = L.malus_std_layernorm_fwd(x, 1, C.byref(v))
        L.tensor_free(v.value)
        return y

    timed("layernorm", 8 * n + 4 * Rr, ln_fwd, "65536x1024")
    timed("layernorm VJP", 12 * n + 4 * Rr, lambda: L.malus_std_layernorm_bwd(ln, var.value, dout, 1), "65536x1024")
    timed("gelu", 8 * n, lambda: L.malus_std_gelu_fwd(x), "65536x1024")
    timed("gelu VJP", 12 * n, lambda: L.malus_std_gelu_bwd(x, dout), "65536x1024")

    def ce_fwd():
        p = C.c_int64()
        l = L.malus_std_cross_entropy_fwd(logits, tg, C.byref(p))
        L.tensor_free(p.value)
        return l

    timed("cross_entropy", 8 * n + 8 * Rr, ce_fwd, "65536x1024")
    timed("cross_entropy VJP", 8 * n + 4 * Rr, lambda: L.malus_std_cross_entropy_bwd(probs.value, tg, one), "65536x1024")
    timed("sum axis 1", 4 * n + 4 * Rr, lambda: L.malus_std_reduce_fwd(M.R_SUM, x, 1, 0), "65536x1024")
    timed("sum axis 0", 4 * n + 4 * V, lambda: L.malus_std_reduce_fwd(M.R_SUM, x, 0, 0), "65536x1024")
    rt.free(x, dout, logits, tg, sm, var.value, ln, probs.value, loss, one)
    return rows


def attention_suite(rt, M, reps: int):
    """Causal attention forward and backward per call: the row-register
    fused kernels (T <= 256) and flash attention (any T multiple of 32), in
    f32 and under autocast, at C5's shape (B*H = 384, T = 256, hs = 64) and
    at longer T with the same tokens per call.  Rate: algorithmic FLOP
    (forward: Q K^T and P V; backward: dP, dQ, dK, dV; causal pairs only,
    2 * hs per query-key pair per product) / time."""
    import numpy as np

    L = rt.L
    rng = np.random.default_rng(5)
    rows = []

    def timed(fn):
        for _ in range(2):
            fn()
        L.gpu_barrier()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        L.gpu_barrier()
        return (time.perf_counter() - t0) / reps

    for bh, t, hs in [(384, 256, 64), (96, 1024, 64), (48, 2048, 64), (24, 4096, 64)]:
        q, k, v, d = (rt.tensor(rng.uniform(-1, 1, (bh, t, hs)).astype(np.float32)) for _ in range(4))
        sc = rt.tensor(np.array([[1.0 / np.sqrt(hs)]], np.float32))
        pairs = bh * t * (t + 1) / 2
        f_fwd, f_bwd = 2 * 2.0 * hs * pairs, 4 * 2.0 * hs * pairs
        for ac in (0, 1):
            prev = L.malus_autocast(ac)
            lse = C.c_int64()
            out = L.malus_std_flash_attn_fwd(q, k, v, sc, 1, C.byref(lse))

            def flash_fwd():
                h = L.malus_std_flash_attn_fwd(q, k, v, sc, 1, None)
                L.tensor_free(h)

            def flash_bwd():
                g = [C.c_int64() for _ in range(3)]
                L.malus_std_flash_attn_bwd(d, q, k, v, out, lse.value, sc, 1, 0, 0, 0, *[C.byref(x) for x in g])
                for x in g:
                    L.tensor_free(x.value)

            tf, tb = timed(flash_fwd), timed(flash_bwd)
            rows.append({"kernel": "flash", "bh": bh, "t": t, "hs": hs, "autocast": bool(ac),
                         "fwd_us": round(tf * 1e6, 1), "bwd_us": round(tb * 1e6, 1),
                         "fwd_TFLOPs": round(f_fwd / tf / 1e12, 1), "bwd_TFLOPs": round(f_bwd / tb / 1e12, 1)})
            L.tensor_free(out)
            L.tensor_free(lse.value)
            if t <= 256 and not ac:
                mask = L.tensor_causal_mask(t)
                p = C.c_int64()
                o2 = L.malus_std_attn_fwd(q, k, v, sc, mask, 1, C.byref(p))

                def rows_fwd():
                    pp = C.c_int64()
                    h = L.malus_std_attn_fwd(q, k, v, sc, mask, 1, C.byref(pp))
                    L.tensor_free(h)
                    L.tensor_free(pp.value)

                def rows_bwd():
                    g = [C.c_int64() for _ in range(3)]
                    ds = L.malus_std_attn_bwd_all(d, q, k, v, p.value, sc, 1, 0, 0, 0, *[C.byref(x) for x in g])
                    L.tensor_free(ds)
                    for x in g:
                        L.tensor_free(x.value)

                tf, tb = timed(rows_fwd), timed(rows_bwd)
                rows.append({"kernel": "rows", "bh": bh, "t": t, "hs": hs, "autocast": False,
                             "fwd_us": round(tf * 1e6, 1), "bwd_us": round(tb * 1e6, 1),
                             "fwd_TFLOPs": round(f_fwd / tf / 1e12, 1), "bwd_TFLOPs": round(f_bwd / tb / 1e12, 1)})
                for h in (mask, p.value, o2):
                    L.tensor_free(h)
            L.malus_autocast(prev)
        for h in (q, k, v, d, sc):
            L.tensor_free(h)
    for r in rows:
        log(f"  {r['kernel']:5s} bh {r['bh']:4d} t {r['t']:5d} hs {r['hs']} {'bf16' if r['autocast'] else 'f32 '}  "
            f"fwd {r['fwd_us']:8.1f} us {r['fwd_TFLOPs']:6.1f} TF/s   bwd {r['bwd_us']:8.1f} us {r['bwd_TFLOPs']:6.1f} TF/s")
    return rows


def host_cpu():
    """The host the CPU baseline ran on: usable cores and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return avail, model


def cpu_baseline(cfg, batches, threads: int):
    """The oracle (plain-C restatement of the reference CPU path) on a
    bounded sample.  One full training step costs a + b*B: the forward and
    backward scale with the batch B, the optimizer and the batch-independent
    parts (AdamW over every parameter, the LN-weight and embedding-table
    sizes) do not.  Time one step at each of two small batches, fit a and b,
    and report the step at the configured batch."""
    from oracle import oracle as O
    import numpy as np

    O.set_threads(threads)
    rng = np.random.default_rng(7)
    pts = []
    for b in batches:
        c = dict(cfg, B=b)
        g = O.Gpt(**c, rng_call_idx=0, **OPT)
        n = b * c["T"]
        x = rng.integers(0, c["V"], n).astype(np.int32)
        y = rng.integers(0, c["V"], n).astype(np.int32)
        t0 = time.perf_counter()
        g.step(x, y, 1)
        pts.append((b, time.perf_counter() - t0))
        del g
    (b0, t0_), (b1, t1_) = pts
    per_b = (t1_ - t0_) / (b1 - b0)
    fixed = t0_ - per_b * b0
    est = fixed + per_b * cfg["B"]
    avail, model = host_cpu()
    return dict(value=round(est * 1e3, 1), unit="ms/step", cores=threads, kind="port",
                cores_available=avail, cpu_model=model,
                method=f"one oracle step at batch {b0} ({t0_:.2f} s) and at batch {b1} ({t1_:.2f} s); "
                       f"fit a + b*B (a = {fixed:.3f} s, b = {per_b:.3f} s per sequence), evaluated at B={cfg['B']}",
                sample=f"2 full steps (batches {b0} and {b1}) of the {cfg['B']}-sequence workload")


def cpu_baseline_xor(steps: int):
    """The oracle's XOR training (examples/xor.ml), all `steps` steps, 1 thread."""
    from oracle import oracle as O

    t0 = time.perf_counter()
    O.xor_train(steps, 1.5)
    dt = time.perf_counter() - t0
    avail, model = host_cpu()
    return dict(value=round(dt * 1e3 / steps, 5), unit="ms/step", cores=1, kind="port", cores_available=avail,
                cpu_model=model, total_s=round(dt, 4), method=f"the full {steps}-step run, timed once",
                sample=f"all {steps} steps")


# examples/xor.ml:1-2 `sigmoid_backward`, the one user kernel on the C1 path,
# lowered to the v1 kernel ABI (implicit form: out[tid] = expr).
SIGMOID_BACKWARD_ML = """kernel sigmoid_backward(grad_out: Tensor<f32>, sig_z: Tensor<f32>) -> Tensor<f32>:
    return grad_out * sig_z * (1.0 - sig_z)
"""


def xor_kernel_id(rt):
    """Lower xor.ml's user kernel with the library's HIP emitter and register
    it through malus_runtime_init; returns its kernel id."""
    import malus_amd as M

    reg = M.compile_kernels(SIGMOID_BACKWARD_ML)
    rt.L.malus_runtime_init(*reg.init_args())
    return reg.ids["sigmoid_backward"]


def run_xor(rt, a):
    """C1: the XOR MLP's 10,000 training steps (examples/xor.ml) through the
    C ABI; every step is ~37 runtime ops on [4,8]-sized tensors, so the
    figure is launch and latency bound (no roofline applies)."""
    L = rt.L
    kid = xor_kernel_id(rt)
    steps = 10000
    loss_at, preds, params = (C.c_float * 6)(), (C.c_float * 4)(), (C.c_float * 33)()
    for _ in range(a.warmup):
        L.malus_xor_run(100, 1.5, kid, None, None, None)
    L.gpu_barrier()
    runs = []
    for _ in range(max(1, min(a.steps, 5))):
        t0 = time.perf_counter()
        loss = L.malus_xor_run(steps, 1.5, kid, loss_at, preds, params)
        L.gpu_barrier()
        runs.append(time.perf_counter() - t0)
    total = statistics.median(runs)
    log(f"xor: {len(runs)} runs of {steps} steps, median {total:.3f} s ({total * 1e3 / steps:.4f} ms/step), "
        f"final loss {loss:.8g}, predictions {[round(v, 6) for v in preds]}")
    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline_xor(steps)
        log(f"cpu baseline: {cpu}")
    return {
        "metric": METRIC, "value": round(total * 1e3 / steps, 5), "unit": "ms/step", "n_gpus": 1,
        "steps": steps, "warmup": a.warmup, "ms_per_step": round(total * 1e3 / steps, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "the fixed tensors of examples/xor.ml (no RNG)",
        "config": {"workload": "C1 XOR MLP 2-8-1, 10,000 SGD steps (lr 1.5)", "total_s": round(total, 4),
                   "runs": len(runs), "final_loss": loss, "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": cpu,
    }


def run_gpt(rt, a, cfg):
    L = rt.L
    import numpy as np

    name = C.create_string_buffer(64)
    cus, clk = C.c_int(), C.c_int()
    L.malus_device_info(name, 64, C.byref(cus), C.byref(clk))
    log(f"device {name.value.decode()} CUs {cus.value} clock {clk.value / 1e6:.2f} GHz")

    L.malus_rng_set_counter(0)
    g = L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"], OPT["b1"],
                           OPT["b2"], OPT["eps"], OPT["wd"])
    L.malus_gpt_set_attention(g, ATTN_MODES[a.attention])
    if a.composed:
        # the op sequence an unchanged nanogpt_modular.ml issues through the C ABI:
        # no forward fusions, the tape's plain VJPs, op-by-op AdamW
        L.malus_gpt_set_fused_forward(g, 0)
        L.malus_gpt_set_fused_optimizer(g, 0)
        L.malus_tape_set_fused_vjps(0)
    if a.f32_activations:
        L.malus_gpt_set_bf16_activations(g, 0)
    # f32 GEMM products: split bf16 pieces on the bf16 MFMA (default) or the FP32 MFMA
    L.malus_gemm_set_f32_split(1 if a.f32_gemm == "split" else 0)
    # docs/adr/0037-bf16-autocast.md:5-12: the whole step inside `with autocast:`
    L.malus_autocast(1 if a.autocast else 0)
    n = cfg["B"] * cfg["T"]
    gemm_steps = 0 if a.no_gemm_pass else min(a.steps, 20)

    t = 0
    graph = None

    def calls(i):
        # step i's token and target ids: rand_int(V) per token with call
        # indices base + j and base + n + j (i.i.d. uniform in [0, V))
        base = (1 << 33) + 2 * n * i
        return base, base + n

    def step(i):
        # batch construction (the ids drawn on the device), then the step
        nonlocal t, graph
        t += 1
        cx, cy = calls(i)
        if a.graph:
            if graph is None:  # step 1 runs eagerly inside create, which then captures the step
                hl = C.c_int64()
                graph = L.malus_gpt_graph_create_drawn(g, cx, cy, t, C.byref(hl))
                if not graph:
                    raise RuntimeError("malus_gpt_graph_create_drawn failed")
                return hl.value, 0, 0
            return L.malus_gpt_graph_step_drawn(graph, cx, cy, t), 0, 0
        x, y = L.malus_rand_tokens_device(cx, n, cfg["V"]), L.malus_rand_tokens_device(cy, n, cfg["V"])
        hl = L.malus_gpt_step(g, x, y, t)
        return hl, x, y

    first_loss = last_loss = None
    for i in range(a.warmup):
        hl, x, y = step(i)
        L.gpu_barrier()
        if first_loss is None:
            first_loss = L.malus_tensor_get_f32(hl, 0)
        rt.free(hl, x, y)
    L.gpu_barrier()

    # headline: the kernel timer is off
    times, enq = [], []
    t_all = time.perf_counter()
    for i in range(a.steps):
        t0 = time.perf_counter()
        hl, x, y = step(a.warmup + i)
        enq.append((time.perf_counter() - t0) * 1e3)
        L.gpu_barrier()  # flush inside the timed step
        times.append((time.perf_counter() - t0) * 1e3)
        if i == a.steps - 1:
            last_loss = L.malus_tensor_get_f32(hl, 0)
        rt.free(hl, x, y)
    L.gpu_barrier()
    wall = time.perf_counter() - t_all
    nodes = 0
    if graph is not None:
        nodes = L.malus_gpt_graph_nodes(graph)
        L.malus_gpt_graph_free(graph)
        graph = None
        log(f"graph: one hipGraphLaunch per step, {nodes} nodes (kernels, the token draw and its input copy)")
    a_graph, a.graph = a.graph, False  # the GEMM pass below runs eagerly (event timers are not graph nodes)

    # a separate pass for the GEMM class: HIP events around every GEMM launch
    L.malus_ktimer_collect(None, C.byref(C.c_double()), C.byref(C.c_double()))  # drop stale records
    L.malus_ktimer_enable(1)
    for i in range(gemm_steps):
        hl, x, y = step(a.warmup + a.steps + i)
        L.gpu_barrier()
        rt.free(hl, x, y)
    L.malus_ktimer_enable(0)
    gms, gflop = C.c_double(), C.c_double()
    ng = L.malus_ktimer_collect(b"gemm", C.byref(gms), C.byref(gflop))

    med = statistics.median(times)
    step_flops = gemm_flops_per_step(cfg)
    gemm_tflops = gflop.value / (gms.value * 1e-3) / 1e12 if gms.value > 0 else 0.0
    gsteps = max(gemm_steps, 1)
    log(f"steps {a.steps}: median {med:.3f} ms  min {min(times):.3f}  max {max(times):.3f}  wall {wall:.2f} s  "
        f"(host enqueue median {statistics.median(enq):.3f} ms)")
    log(f"loss first {first_loss:.4f} last {last_loss:.4f}")
    ps = (C.c_int64 * 4)()
    L.malus_pool_stats(ps)
    log(f"pool: hits {ps[0]} misses {ps[1]} peak device bytes {ps[3] / 1e9:.2f} GB")
    log(f"gemm ({gemm_steps} separate steps): {ng} launches, {gms.value / gsteps:.3f} ms/step, "
        f"{gemm_tflops:.1f} TFLOP/s ({gflop.value / gsteps / 1e9:.1f} GFLOP/step; "
        f"algorithmic {step_flops / 1e9:.1f})")

    cpu = None
    if not a.no_cpu_baseline:
        try:
            cpu = cpu_baseline(cfg, (1, 2) if cfg["B"] >= 16 else (1, cfg["B"]), a.cpu_threads)
            log(f"cpu baseline: {cpu}")
        except Exception as e:  # the CPU leg is a reported baseline only
            log(f"cpu baseline failed: {e!r}")
    L.malus_gpt_free(g)
    L.malus_autocast(0)
    L.malus_tape_set_fused_vjps(1)

    c5 = cfg == CONFIGS["c5"]
    traffic = measured_traffic() if c5 and not a.autocast else None
    peak = PEAK_BF16_MFMA_TFLOPS if a.autocast else PEAK_FP32_MFMA_TFLOPS
    tag = "C5 Karpathy" if c5 else "C4 toy"
    split = not a.autocast and a.f32_gemm == "split"
    if split:
        # every f32 product of the LDS-DMA GEMMs runs six exact bf16 piece
        # products on the bf16 MFMA; the register-staged launches (the three
        # 65-wide vocabulary products: logits, their dX and dW, 6 n V C FLOP)
        # run on the FP32 MFMA
        gf = gflop.value / gsteps / 1e9
        vocab = 6.0 * n * cfg["V"] * cfg["C"] / 1e9
        exec_tflops = gemm_tflops * (6.0 * (gf - vocab) + vocab) / gf if gf > vocab else gemm_tflops
        executed = {"pipe": "bf16 MFMA (v_mfma_f32_32x32x16_bf16), six piece products per f32 product",
                    "achieved": round(exec_tflops, 2), "peak": PEAK_BF16_MFMA_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(exec_tflops / PEAK_BF16_MFMA_TFLOPS, 4)}
    f32_gemm = ("split: each f32 operand value as three exact bf16 pieces, six piece products per f32 product "
                "on the bf16 MFMA, f32 accumulation (error vs float64 no larger than the FP32 MFMA's)") if split \
        else "FP32 MFMA (v_mfma_f32_32x32x2_f32)" if not a.autocast else None
    return {
        "metric": METRIC,
        "value": round(med, 3),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(med, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16 GEMM and attention operands, f32 accumulation; the activations read only as bf16 operands "
                  "stored in bf16 (layernorm-scale outputs, gelu(h), dh, q, k, v and their gradients) and bf16 "
                  "copies of the block weights as GEMM operands; everything else f32 (autocast)")
                 if a.autocast and not a.f32_activations else
                 "bf16 GEMM operands, f32 accumulation and everything else f32 (autocast)" if a.autocast else "f32",
        "f32_gemm": f32_gemm,
        "data": "synthetic int32 tokens i.i.d. uniform in [0,65), drawn on the device inside each timed step "
                "(rand_int per token, Philox keyed by call index); weights randn*0.02 (Philox, call 0)",
        "attention": a.attention,
        "execution": ("hipGraph replay of the captured step (the id draw, the step's call indices and AdamW bias "
                      f"corrections from pinned host memory by the graph's nodes; {nodes} nodes)") if a_graph else
                     "eager: every kernel launched from the host each step",
        "ops": ("composed: nanogpt_modular.ml's op sequence through the C ABI (no forward fusions, plain tape VJPs, "
                "op-by-op AdamW)") if a.composed else "fused forward, fused VJPs, multi-tensor AdamW",
        "config": {"workload": f"{tag} char-nanoGPT train step (batch draw+fwd+bwd+AdamW)", "vocab": cfg["V"],
                   "block_size": cfg["T"], "n_embd": cfg["C"], "n_head": cfg["H"], "n_layer": cfg["L"],
                   "batch": cfg["B"], "tokens_per_step": n, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "k_sgemm (all GEMM launches of the step)",
                     "achieved": round(gemm_tflops, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / peak, 4), "traffic": traffic,
                     "traffic_unit": "HBM bytes per step, all GEMM launches (rocprofv3 FETCH_SIZE+WRITE_SIZE)",
                     "algorithmic_bytes": gemm_bytes_per_step(cfg),
                     "timing": f"HIP events around each GEMM launch over {gemm_steps} steps run after the "
                               "headline steps (the headline runs with the event timer off)",
                     "gemm_ms_per_step": round(gms.value / gsteps, 3),
                     "gemm_gflop_per_step": round(gflop.value / gsteps / 1e9, 1),
                     **({"note": "achieved counts the f32 product's FLOPs (2 M N K per launch) against the FP32 MFMA "
                                 "peak, the bar the f32 matmul is held to; executed: the bf16 MFMA work the split "
                                 "products run, against that pipe's peak",
                         "executed": executed} if split else {})},
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", choices=["c5", "c4", "c1"], default="c5",
                    help="c5 (default): Karpathy char-nanoGPT; c4: toy char-nanoGPT; c1: XOR MLP, 10,000 steps")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel of the step from the host (default: the step captured once as a "
                         "hipGraph and replayed, malus_gpt_graph_*, with each step's tokens copied in by its nodes)")
    ap.add_argument("--autocast", action="store_true",
                    help="run the step in the bf16 autocast scope (bf16 GEMMs, f32 accumulation, f32 master state); "
                         "reported alongside the f32 headline, never in its place")
    ap.add_argument("--attention", choices=list(ATTN_MODES), default="auto",
                    help="attention kernel of the model: auto, flash (online softmax), rows (the row-register "
                         "fused kernel), composed (matmul + softmax ops)")
    ap.add_argument("--composed", action="store_true",
                    help="the op sequence an unchanged nanogpt_modular.ml issues through the C ABI: forward fusions, "
                         "fused VJPs and the fused optimizer off, composed attention, eager launches; reported "
                         "beside the headline, never in its place")
    ap.add_argument("--f32-gemm", choices=["split", "fp32"], default="split",
                    help="f32 GEMM products: split (default; each operand value as three exact bf16 pieces, six "
                         "piece products on the bf16 MFMA with f32 accumulation) or fp32 (the FP32 MFMA)")
    ap.add_argument("--f32-activations", action="store_true",
                    help="with --autocast: keep every activation and weight operand in f32 (the same values; for "
                         "comparison with the default bf16 storage of what only bf16 products read)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-gemm-pass", action="store_true",
                    help="skip the event-timed eager GEMM pass after the headline steps (for a kernel trace of the "
                         "headline steps alone; the roofline figures are then empty)")
    ap.add_argument("--cpu-threads", type=int, default=1)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB copy (counter calibration for the traffic figure)")
    ap.add_argument("--suite", choices=["kernels", "attention"],
                    help="kernels: the C2/C3 elementwise and row-op kernels' HBM bandwidth; attention: the causal "
                         "attention kernels' forward and backward times (one JSON line each)")
    a = ap.parse_args()
    if a.composed:
        a.eager, a.attention = True, "composed"
    a.graph = not a.eager
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU data parallelism is designed but not built", file=sys.stderr)
        sys.exit(2)

    import malus_amd as M

    rt = M.Runtime()
    if a.copy_calibration:
        copy_calibration(rt, M.sizes)
        return
    if a.suite == "kernels":
        rows = kernel_suite(rt, M, reps=10)
        print(json.dumps({"suite": "kernels", "unit": "GB/s", "peak_hbm_GBs": PEAK_HBM_GBS, "rows": rows}), flush=True)
        return
    if a.suite == "attention":
        rows = attention_suite(rt, M, reps=10)
        print(json.dumps({"suite": "attention", "peak_fp32_TFLOPs": PEAK_FP32_MFMA_TFLOPS,
                          "peak_bf16_TFLOPs": PEAK_BF16_MFMA_TFLOPS, "rows": rows}), flush=True)
        return
    out = run_xor(rt, a) if a.config == "c1" else run_gpt(rt, a, CONFIGS[a.config])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
