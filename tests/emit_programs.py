"""Kernel programs in the malus kernel language for the HIP emitter's tests.

Written for these tests: together they use every construct the emitter
lowers (implicit maps; explicit bodies with thread intrinsics, `let shared`
arrays, `barrier()`, while/for/if-else, `t.shape[k]`, `t.strides[k]`,
`t.ndim`, multi-index reads, i32/f32 uniforms, an i32 output, `**`, the
math builtins and `and`/`or`/`not`).  Shared by the CPU tests (emitted text,
hipRTC compilation) and the GPU tests (launches against the oracle).
"""

# The XOR workload's user kernel (examples/xor.ml): the backward of a
# sigmoid, g * s * (1 - s), as an implicit map.
SIGMOID_BACKWARD = """kernel sigmoid_backward(grad_out: Tensor<f32>, sig_z: Tensor<f32>) -> Tensor<f32>:
    return grad_out * sig_z * (1.0 - sig_z)
"""

PROGRAM = '''
# an implicit map with a let binding
kernel axpb(x: Tensor<f32>, y: Tensor<f32>) -> Tensor<f32>:
    let twice = x + x
    return twice * y - -x

# one element of x moved by delta (the gradient-check perturbation)
kernel nudge(x: Tensor<f32>, at: i32, delta: f32) -> Tensor<f32>:
    let i = thread_id()
    let mut v = x[i]
    if i == at:
        v = v + delta
    out[i] = v

# row softmax: one workgroup per row of `ncols` (a power of two <= 1024),
# tree reductions in shared memory for the max and the sum
kernel row_softmax(x: Tensor<f32>, ncols: i32) -> Tensor<f32>:
    let row = threadgroup_id()
    let lane = thread_in_threadgroup()
    let width = threads_per_threadgroup()
    let shared vals: Array<f32, 1024>
    let shared red: Array<f32, 1024>
    let v = x[row * ncols + lane]
    vals[lane] = v
    red[lane] = v
    barrier()
    let mut stride = width / 2
    while stride > 0:
        if lane < stride:
            red[lane] = fmax(red[lane], red[lane + stride])
        barrier()
        stride = stride / 2
    let m = red[0]
    barrier()
    let e = exp(vals[lane] - m)
    red[lane] = e
    barrier()
    stride = width / 2
    while stride > 0:
        if lane < stride:
            red[lane] = red[lane] + red[lane + stride]
        barrier()
        stride = stride / 2
    out[row * ncols + lane] = e / red[0]

# a - b with b broadcast NumPy-style onto a (right-aligned, size-1 dims)
kernel bcast_sub(a: Tensor<f32>, b: Tensor<f32>) -> Tensor<f32>:
    let flat = thread_id()
    let lead = a.ndim - b.ndim
    let mut rem = flat
    let mut boff = 0
    for d in range(0, a.ndim):
        let q = rem / a.strides[d]
        rem = rem - q * a.strides[d]
        if d >= lead and b.shape[d - lead] > 1:
            boff = boff + q * b.strides[d - lead]
    out[flat] = a[flat] - b[boff]

# 2-D transpose through a multi-index read
kernel transpose2(x: Tensor<f32>) -> Tensor<f32>:
    let flat = thread_id()
    let rows = x.shape[0]
    let c = flat / rows
    let r = flat - c * rows
    out[flat] = x[r, c]

# rows of a table gathered by i32 indices; out-of-range rows read as zeros
kernel gather_rows(table: Tensor<f32>, idx: Tensor<i32>, dim: i32, nrows: i32) -> Tensor<f32>:
    let flat = thread_id()
    let t = flat / dim
    let c = flat - t * dim
    let row = idx[t]
    if row < 0 or row >= nrows:
        out[flat] = 0.0
    else:
        out[flat] = table[row * dim + c]

# the sum down each column, rows in order
kernel col_sum(x: Tensor<f32>, nrows: i32) -> Tensor<f32>:
    let c = thread_id()
    let ncols = x.shape[1]
    let mut s = 0.0
    let mut r = 0
    while r < nrows:
        s = s + x[r * ncols + c]
        r = r + 1
    out[c] = s

# the first index of each row's maximum, as an i32 tensor
kernel row_argmax(x: Tensor<f32>, ncols: i32) -> Tensor<i32>:
    let row = thread_id()
    let mut best = x[row * ncols]
    let mut at = 0
    for c in range(1, ncols):
        let v = x[row * ncols + c]
        if v > best:
            best = v
            at = c
    out[row] = at

# every scalar math builtin, ** and the logical operators
kernel math_mix(x: Tensor<f32>, y: Tensor<f32>, k: f32) -> Tensor<f32>:
    let i = thread_id()
    let a = x[i]
    let b = y[i]
    let mut r = tanh(a) * k + sigmoid(b) - relu(-a)
    r = r + abs(b) ** 1.5 + fmin(a, b) / fmax(sqrt(abs(a)) + 1.0, rsqrt(b * b + 1.0))
    if not (a > 0.0) and b < 0.0:
        r = r + log(1.0 + a * a)
    else:
        if a > b or b == 0.0:
            r = r - exp(-a * b)
    out[i] = r
'''

# every synthesized builtin (codegen-gpu/lib.rs:373-418)
BUILTINS = ["malus_add", "malus_sub", "malus_mul", "malus_div", "malus_add_scalar", "malus_sub_scalar",
            "malus_rsub_scalar", "malus_mul_scalar", "malus_div_scalar", "malus_rdiv_scalar",
            "relu", "sigmoid", "tanh", "exp", "log", "sqrt", "abs"]
