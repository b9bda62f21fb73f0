/*
 * malus CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Sequential host-f32 restatement of the reference runtime.  Compiled with
 * -ffp-contract=off so every f32 operation rounds exactly once, like Rust's
 * f32 arithmetic in the reference.  Loops that the reference runs
 * sequentially are sequential here; OpenMP only splits independent output
 * elements (GEMM rows), which leaves every per-element summation order
 * unchanged.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }

static void die(const char* msg) {
    fprintf(stderr, "malus-oracle: %s\n", msg);
    abort();
}

static size_t prod(const size_t* s, int n) {
    size_t p = 1;
    for (int i = 0; i < n; ++i) p *= s[i];
    return p;
}

/* ========================================================================
 * Philox4x32-10 and the RNG builtins — metal.rs:1690-1759
 * ====================================================================== */
#define PHILOX_M0 0xD2511F53u /* metal.rs:1692 */
#define PHILOX_M1 0xCD9E8D57u /* metal.rs:1693 */
#define PHILOX_W0 0x9E3779B9u /* metal.rs:1694 */
#define PHILOX_W1 0xBB67AE85u /* metal.rs:1695 */

void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    /* metal.rs:1702-1711: ten rounds, key bumped after every round. */
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)c0 * PHILOX_M0;
        uint64_t p1 = (uint64_t)c2 * PHILOX_M1;
        uint32_t h0 = (uint32_t)(p0 >> 32), l0 = (uint32_t)p0;
        uint32_t h1 = (uint32_t)(p1 >> 32), l1 = (uint32_t)p1;
        uint32_t n0 = h1 ^ c1 ^ k0, n1 = l1, n2 = h0 ^ c3 ^ k1, n3 = l0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

void or_randn(uint64_t call_idx, size_t n, float* out) {
    /* metal.rs:1720-1740: key = call index, counter = pair index,
     * Box-Muller in f64, each value cast to f32. */
    uint32_t key[2] = {(uint32_t)call_idx, (uint32_t)(call_idx >> 32)};
    size_t n_pairs = (n + 1) / 2;
    const double two_pi = 2.0 * 3.14159265358979311599796346854; /* std::f64::consts::PI */
    for (size_t k = 0; k < n_pairs; ++k) {
        uint32_t ctr[4] = {(uint32_t)k, (uint32_t)((uint64_t)k >> 32), 0u, 0u};
        uint32_t r[4];
        or_philox4x32_10(ctr, key, r);
        double u1 = ((double)r[0] + 0.5) / 4294967296.0;
        double u2 = ((double)r[1] + 0.5) / 4294967296.0;
        double mag = sqrt(-2.0 * log(u1));
        out[2 * k] = (float)(mag * cos(two_pi * u2));
        if (2 * k + 1 < n) out[2 * k + 1] = (float)(mag * sin(two_pi * u2));
    }
}

float or_rand_uniform(uint64_t call_idx) {
    /* metal.rs:1744-1750: counter 0, r0 / 2^32 in f64, then f32. */
    uint32_t key[2] = {(uint32_t)call_idx, (uint32_t)(call_idx >> 32)};
    uint32_t ctr[4] = {0, 0, 0, 0}, r[4];
    or_philox4x32_10(ctr, key, r);
    return (float)((double)r[0] / 4294967296.0);
}

int64_t or_rand_int(uint64_t call_idx, int64_t n) {
    /* metal.rs:1752-1759: counter[0] = 1, r0 mod n. */
    uint32_t key[2] = {(uint32_t)call_idx, (uint32_t)(call_idx >> 32)};
    uint32_t ctr[4] = {1, 0, 0, 0}, r[4];
    or_philox4x32_10(ctr, key, r);
    return (int64_t)((uint64_t)r[0] % (uint64_t)n);
}

void or_rand_tokens(uint64_t call_idx, size_t n, int64_t vocab, int32_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (int32_t)or_rand_int(call_idx + i, vocab);
}

/* ========================================================================
 * Elementwise ops
 * ====================================================================== */
static float apply_op(int op, float x, float y) {
    switch (op) {
    case OR_ADD: return x + y;
    case OR_SUB: return x - y;
    case OR_MUL: return x * y;
    case OR_DIV: return x / y;
    }
    die("bad binop");
    return 0.f;
}

/* NumPy right-aligned broadcast of (first op second), first index from the
 * output index (metal.rs:1021-1073 broadcast_result_shape/broadcast_cpu_loop).
 * The operand swap of __broadcast_<op>_fwd (broadcast_binop.ml:82-112) is
 * applied first: when a.ndim < b.ndim the kernel computes b op a. */
void or_broadcast_fwd(int op, const float* a, const size_t* ash, int and_,
                      const float* b, const size_t* bsh, int bnd,
                      float* out, size_t* out_shape, int* out_ndim) {
    const float *p = a, *q = b;
    const size_t *ps = ash, *qs = bsh;
    int pn = and_, qn = bnd;
    if (and_ < bnd) { /* broadcast_binop.ml:86-88 */
        p = b; ps = bsh; pn = bnd;
        q = a; qs = ash; qn = and_;
    }
    int n = pn; /* pn >= qn */
    size_t pp[8], qq[8], os[8];
    for (int i = 0; i < n; ++i) {
        pp[i] = ps[i];
        qq[i] = (i >= n - qn) ? qs[i - (n - qn)] : 1;
        if (pp[i] == qq[i] || qq[i] == 1) os[i] = pp[i];
        else if (pp[i] == 1) os[i] = qq[i];
        else die("broadcast shape mismatch");
    }
    size_t total = prod(os, n);
    for (size_t flat = 0; flat < total; ++flat) {
        size_t rem = flat, idx[8];
        for (int d = n - 1; d >= 0; --d) { idx[d] = rem % os[d]; rem /= os[d]; }
        size_t pf = 0, qf = 0;
        for (int d = 0; d < n; ++d) {
            pf = pf * pp[d] + (idx[d] % pp[d]);
            qf = qf * qq[d] + (idx[d] % qq[d]);
        }
        out[flat] = apply_op(op, p[pf], q[qf]);
    }
    for (int i = 0; i < n; ++i) out_shape[i] = os[i];
    *out_ndim = n;
}

/* codegen-gpu/lib.rs:400-418 synthesize_scalar_builtin */
void or_scalar_op(int op, int scalar_on_right, const float* a, size_t n, float s, float* out) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < n; ++i)
        out[i] = scalar_on_right ? apply_op(op, a[i], s) : apply_op(op, s, a[i]);
}

/* tensor_gelu, metal.rs:1535-1549 (C0, C1 and the expression order). */
static float gelu_f(float x) {
    const float C0 = 0.7978845608f, C1 = 0.044715f;
    float inner = C0 * (x + C1 * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* codegen-gpu/lib.rs:375-381 synthesize_unary_builtin; gelu per above.
 * exp / log / tanh (also inside sigmoid) are the correctly rounded f32
 * functions: evaluated in double and rounded once.  The reference's host f32
 * calls go to the platform libm (Apple's on its Metal hosts, glibc here),
 * which is within 1 ulp but not correctly rounded; the sigmoid formula
 * amplifies that last-bit choice (1 + e rounds at e's spacing), so the
 * platform-independent correctly rounded functions are the restatement. */
void or_unary(int op, const float* a, size_t n, float* out) {
    if (op < OR_RELU || op > OR_GELU) die("bad unary op");
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float x = a[i];
        switch (op) {
        case OR_RELU: out[i] = fmaxf(0.0f, x); break;
        case OR_SIGMOID: out[i] = 1.0f / (1.0f + (float)exp(-(double)x)); break;
        case OR_TANH: out[i] = (float)tanh((double)x); break;
        case OR_EXP: out[i] = (float)exp((double)x); break;
        case OR_LOG: out[i] = (float)log((double)x); break;
        case OR_SQRT: out[i] = sqrtf(x); break;
        case OR_ABS: out[i] = fabsf(x); break;
        default: out[i] = gelu_f(x); break; /* OR_GELU */
        }
    }
}

/* ========================================================================
 * Reductions — metal.rs:1124-1271 (sequential along the axis)
 * ====================================================================== */
static void outer_axis_inner(const size_t* shape, int ndim, int axis, size_t* o, size_t* a, size_t* in) {
    if (axis < 0) axis += ndim; /* normalize_axis, metal.rs:1124-1131 */
    if (axis < 0 || axis >= ndim) die("axis out of range");
    *o = prod(shape, axis);
    *a = shape[axis];
    *in = prod(shape + axis + 1, ndim - axis - 1);
}

void or_reduce_axis(int op, const float* x, const size_t* shape, int ndim, int axis, float* out) {
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
    for (size_t o = 0; o < O; ++o)
        for (size_t i = 0; i < I; ++i) {
            const float* base = x + o * A * I + i;
            float r;
            if (op == OR_RMAX) { /* metal.rs:1208-1222, NEG_INFINITY + f32::max */
                r = -INFINITY;
                for (size_t k = 0; k < A; ++k) r = fmaxf(r, base[k * I]);
            } else {
                float s = 0.0f;
                for (size_t k = 0; k < A; ++k) s += base[k * I];
                if (op == OR_RSUM) r = s;
                else {
                    float mean = s / (float)A; /* metal.rs:1201 */
                    if (op == OR_RMEAN) r = mean;
                    else { /* metal.rs:1240-1268 population variance */
                        float v = 0.0f;
                        for (size_t k = 0; k < A; ++k) { float d = base[k * I] - mean; v += d * d; }
                        r = v / (float)A;
                    }
                }
            }
            out[o * I + i] = r;
        }
}

/* VJPs of the axis reductions: tape.rs:1085-1145, composed the same way by
 * reduce_bwd.ml:40-71.  y is the forward output (used by max only); dout
 * has outer*inner elements.
 *   sum:  dx = expand(dout)
 *   mean: dx = expand(dout * (1/n))                    (scalar_mul, 1.0/n)
 *   max:  dx = expand(dout) * (x == expand(y))         (every tied max gets it)
 *   var:  dx = expand(dout) * ((x - expand(mean)) * (2/n)), mean keepdim     */
void or_reduce_axis_bwd(int op, const float* x, const float* y, const float* dout, const size_t* shape, int ndim,
                        int axis, float* out) {
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
    float* mean = NULL;
    if (op == OR_RVAR) {
        mean = (float*)malloc(O * I * sizeof(float));
        or_reduce_axis(OR_RMEAN, x, shape, ndim, axis, mean);
    }
    const float inv_n = 1.0f / (float)A, two_n = 2.0f / (float)A;
    for (size_t o = 0; o < O; ++o)
        for (size_t k = 0; k < A; ++k)
            for (size_t i = 0; i < I; ++i) {
                size_t f = (o * A + k) * I + i, s = o * I + i;
                float r;
                switch (op) {
                case OR_RSUM: r = dout[s]; break;
                case OR_RMEAN: r = dout[s] * inv_n; break;
                case OR_RMAX: r = dout[s] * (x[f] == y[s] ? 1.0f : 0.0f); break;
                default: r = dout[s] * ((x[f] - mean[s]) * two_n); break;
                }
                out[f] = r;
            }
    free(mean);
}

float or_sum_all(const float* x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i];
    return s;
}

/* ========================================================================
 * Softmax / layernorm / cross-entropy / embedding — metal.rs:1437-1688
 * ====================================================================== */
void or_softmax_axis(const float* x, const size_t* shape, int ndim, int axis, float* out) {
    /* softmax_axis_cpu, metal.rs:1439-1467 */
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (size_t o = 0; o < O; ++o)
        for (size_t i = 0; i < I; ++i) {
            const float* xb = x + o * A * I + i;
            float* ob = out + o * A * I + i;
            float mx = -INFINITY;
            for (size_t k = 0; k < A; ++k) if (xb[k * I] > mx) mx = xb[k * I];
            float sum = 0.0f;
            for (size_t k = 0; k < A; ++k) { float e = expf(xb[k * I] - mx); ob[k * I] = e; sum += e; }
            for (size_t k = 0; k < A; ++k) ob[k * I] /= sum;
        }
}

void or_layernorm_axis(const float* x, const size_t* shape, int ndim, int axis, float* out, float* var_out) {
    /* tensor_layernorm_axis, metal.rs:1486-1533: (x - mu) / sqrt(var + 1e-5). */
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (size_t o = 0; o < O; ++o)
        for (size_t i = 0; i < I; ++i) {
            const float* xb = x + o * A * I + i;
            float* ob = out + o * A * I + i;
            float mu = 0.0f;
            for (size_t k = 0; k < A; ++k) mu += xb[k * I];
            mu /= (float)A;
            float va = 0.0f;
            for (size_t k = 0; k < A; ++k) { float d = xb[k * I] - mu; va += d * d; }
            va /= (float)A;
            float sigma = sqrtf(va + 1e-5f);
            if (var_out) var_out[o * I + i] = va;
            for (size_t k = 0; k < A; ++k) ob[k * I] = (xb[k * I] - mu) / sigma;
        }
}

float or_cross_entropy(const float* logits, size_t n, size_t c, const int32_t* targets, float* probs_out) {
    /* tensor_cross_entropy, metal.rs:1555-1598 */
    size_t sh[2] = {n, c};
    float* sm = probs_out ? probs_out : (float*)malloc(n * c * sizeof(float));
    or_softmax_axis(logits, sh, 2, 1, sm);
    float loss = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        int32_t t = targets[i];
        if (t < 0 || (size_t)t >= c) die("cross_entropy target out of range");
        loss -= logf(sm[i * c + (size_t)t]);
    }
    loss /= (float)n;
    if (!probs_out) free(sm);
    return loss;
}

void or_embedding(const float* w, size_t vocab, size_t dim, const int32_t* idx, size_t t, float* out) {
    /* tensor_embedding, metal.rs:1627-1660 */
    for (size_t i = 0; i < t; ++i) {
        int32_t r = idx[i];
        if (r < 0 || (size_t)r >= vocab) die("embedding index out of range");
        memcpy(out + i * dim, w + (size_t)r * dim, dim * sizeof(float));
    }
}

void or_causal_mask(size_t t, float* out) {
    /* tensor_causal_mask, metal.rs:1600-1612 */
    for (size_t i = 0; i < t; ++i)
        for (size_t j = 0; j < t; ++j) out[i * t + j] = (j > i) ? -1e9f : 0.0f;
}

void or_permute(const float* x, const size_t* shape, int ndim, const size_t* perm, float* out) {
    /* permute_by_perm, metal.rs:1346-1382: out[flat] = x[source index of
     * flat].  A pure copy, so visiting the output rows in parallel, with the
     * source offset computed once per row, gives the same result. */
    if (ndim <= 0) { out[0] = x[0]; return; }
    size_t in_st[8], os[8];
    in_st[ndim - 1] = 1;
    for (int i = ndim - 2; i >= 0; --i) in_st[i] = in_st[i + 1] * shape[i + 1];
    for (int d = 0; d < ndim; ++d) os[d] = shape[perm[d]];
    size_t total = prod(os, ndim);
    size_t inner = os[ndim - 1], step = in_st[perm[ndim - 1]];
    if (total == 0) return;
    size_t rows = total / inner;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t row = 0; row < rows; ++row) {
        size_t rem = row, in_flat = 0;
        for (int d = ndim - 2; d >= 0; --d) {
            size_t id = rem % os[d];
            rem /= os[d];
            in_flat += id * in_st[perm[d]];
        }
        float* o = out + row * inner;
        for (size_t j = 0; j < inner; ++j) o[j] = x[in_flat + j * step];
    }
}

/* tensor_matmul_cpu, metal.rs:698-800: out[i,j] accumulates a[i,k]*b[k,j]
 * in k order from 0.0, each product and each sum rounded to f32.
 *
 * The loops below keep that per-element sequence exactly and only change
 * which elements are in flight together: a 4-row x 32-column tile of out is
 * held in 16 eight-float vectors while k runs 0..K-1 (GCC vector extensions:
 * a vector multiply and a vector add are eight independent f32 roundings,
 * and -ffp-contract=off keeps them unfused).  Rows and columns that do not
 * fill a tile take the scalar loop with the same order.  Tiles are split
 * over OpenMP threads by column panel, so a K x 32 panel of b stays in the
 * core's cache while its row tiles pass. */
typedef float v8f __attribute__((vector_size(32)));
#define MM_TR 6
#define MM_TC 16

static void mm_scalar(const float* a, const float* b, float* c, size_t k, size_t n,
                      size_t i0, size_t i1, size_t j0, size_t j1) {
    for (size_t i = i0; i < i1; ++i)
        for (size_t j = j0; j < j1; ++j) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; ++kk) acc += a[i * k + kk] * b[kk * n + j];
            c[i * n + j] = acc;
        }
}

static void mm_tile(const float* a, const float* b, float* c, size_t k, size_t n, size_t i0, size_t j0) {
    v8f acc[MM_TR][MM_TC / 8];
#pragma GCC unroll 8
    for (int r = 0; r < MM_TR; ++r)
#pragma GCC unroll 4
        for (int q = 0; q < MM_TC / 8; ++q) acc[r][q] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
    const float* a0 = a + i0 * k;
    for (size_t kk = 0; kk < k; ++kk) {
        v8f bv[MM_TC / 8];
#pragma GCC unroll 4
        for (int q = 0; q < MM_TC / 8; ++q) memcpy(&bv[q], b + kk * n + j0 + 8 * q, sizeof(v8f));
#pragma GCC unroll 8
        for (int r = 0; r < MM_TR; ++r) {
            float s = a0[r * k + kk];
            v8f av = {s, s, s, s, s, s, s, s};
#pragma GCC unroll 4
            for (int q = 0; q < MM_TC / 8; ++q) acc[r][q] += av * bv[q];
        }
    }
#pragma GCC unroll 8
    for (int r = 0; r < MM_TR; ++r)
#pragma GCC unroll 4
        for (int q = 0; q < MM_TC / 8; ++q) memcpy(c + (i0 + r) * n + j0 + 8 * q, &acc[r][q], sizeof(v8f));
}

/* One [m,k] @ [k,n] product, as tasks of (column panel, 512-row chunk);
 * `par` splits them over threads (callers that already run batches in
 * parallel pass 0). */
static void mm_seq(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int par) {
    const size_t rc = 512;
    size_t nt = n / MM_TC * MM_TC, npan = nt / MM_TC;
    size_t nrc = (m + rc - 1) / rc, ntask = nrc * (npan + 1);
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 1) if (par)
    for (size_t t = 0; t < ntask; ++t) {
        size_t p = t / nrc, i0 = t % nrc * rc;
        size_t i1 = i0 + rc < m ? i0 + rc : m;
        size_t it = i0 + (i1 - i0) / MM_TR * MM_TR;
        if (p < npan) {
            for (size_t i = i0; i < it; i += MM_TR) mm_tile(a, b, c, k, n, i, p * MM_TC);
            mm_scalar(a, b, c, k, n, it, i1, p * MM_TC, (p + 1) * MM_TC);
        } else if (nt < n) {
            mm_scalar(a, b, c, k, n, i0, i1, nt, n);
        }
    }
}

static void mm_rows(const float* a, const float* b, float* c, size_t m, size_t k, size_t n) {
    mm_seq(a, b, c, m, k, n, g_threads > 1);
}

void or_matmul(const float* a, const size_t* ash, int and_, const float* b, const size_t* bsh, int bnd, float* out) {
    if (and_ == 2 && bnd == 2) {
        if (ash[1] != bsh[0]) die("matmul shape mismatch");
        mm_rows(a, b, out, ash[0], ash[1], bsh[1]);
    } else if (and_ == 3 && bnd == 3) {
        if (ash[0] != bsh[0] || ash[2] != bsh[1]) die("batched matmul shape mismatch");
        size_t B = ash[0], m = ash[1], k = ash[2], n = bsh[2];
        /* batches are independent: one batch per worker */
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 1)
        for (size_t bx = 0; bx < B; ++bx) mm_seq(a + bx * m * k, b + bx * k * n, out + bx * m * n, m, k, n, 0);
    } else if (and_ == 3 && bnd == 2) {
        if (ash[2] != bsh[0]) die("matmul shape mismatch");
        mm_rows(a, b, out, ash[0] * ash[1], ash[2], bsh[1]);
    } else {
        die("matmul requires (2,2), (3,3) or (3,2) ranks");
    }
}

/* ========================================================================
 * VJP helpers — metal.rs:1779-1856 and tape.rs cpu_fallback (971-1260)
 * ====================================================================== */
void or_sum_to_shape(const float* g, const size_t* gsh, int gnd, const size_t* tsh, int tnd, float* out) {
    /* sum_to_shape, metal.rs:1812-1842: flat-order accumulation.  Each output
     * element starts at 0.0 and adds its input elements in increasing flat
     * order; here every output element walks its own inputs in that order
     * (the reduced dimensions as an odometer), so elements run in parallel. */
    size_t padded[8], gst[8];
    int rd[8], nr = 0;
    for (int i = 0; i < gnd - tnd; ++i) padded[i] = 1;
    for (int i = 0; i < tnd; ++i) padded[gnd - tnd + i] = tsh[i];
    for (int d = gnd - 1; d >= 0; --d) gst[d] = d == gnd - 1 ? 1 : gst[d + 1] * gsh[d + 1];
    size_t rcount = 1;
    for (int d = 0; d < gnd; ++d)
        if (padded[d] == 1 && gsh[d] > 1) { rd[nr++] = d; rcount *= gsh[d]; }
    size_t outn = prod(tsh, tnd);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t o = 0; o < outn; ++o) {
        size_t rem = o, base = 0;
        for (int d = gnd - 1; d >= 0; --d) { base += (rem % padded[d]) * gst[d]; rem /= padded[d]; }
        float acc = 0.0f;
        for (size_t r = 0; r < rcount; ++r) {
            size_t rr = r, off = base;
            for (int q = nr - 1; q >= 0; --q) { off += (rr % gsh[rd[q]]) * gst[rd[q]]; rr /= gsh[rd[q]]; }
            acc += g[off];
        }
        out[o] = acc;
    }
}

/* Unary VJPs, tape.rs:1041-1083.  x_or_y is the forward output for
 * sigmoid/tanh/exp/sqrt and the forward input for relu/log/abs/gelu. */
void or_unary_bwd(int op, const float* xy, const float* dout, size_t n, float* out) {
    const float C0 = 0.7978845608f, C1 = 0.044715f;
    if (op < OR_RELU || op > OR_GELU) die("bad unary bwd op");
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float v = xy[i], d = dout[i];
        switch (op) {
        case OR_SIGMOID: { float oms = 1.0f - v; float t = d * v; out[i] = t * oms; break; } /* 1041-1048 */
        case OR_RELU: out[i] = d * (v > 0.0f ? 1.0f : 0.0f); break;                       /* 1049-1054 */
        case OR_TANH: out[i] = d * (1.0f - v * v); break;                                 /* 1055-1060 */
        case OR_EXP: out[i] = d * v; break;                                               /* 1061 */
        case OR_LOG: out[i] = d / v; break;                                               /* 1062 */
        case OR_SQRT: { float two_s = v * 2.0f; out[i] = d / two_s; break; }              /* 1063-1068 */
        case OR_ABS: out[i] = d * (v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f)); break;   /* 1069-1074 */
        default: {                                                                        /* GELU, 1187-1199 */
            float g = C0 * (v + C1 * v * v * v);
            float t = tanhf(g);
            float gp = C0 * (1.0f + 3.0f * C1 * v * v);
            float deriv = 0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * gp;
            out[i] = d * deriv;
            break;
        }
        }
    }
}

void or_softmax_bwd(const float* s, const float* dout, const size_t* shape, int ndim, int axis, float* out) {
    /* tape.rs:1150-1161: dx = s * (dout - sum(dout*s, axis, keepdim)) */
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (size_t o = 0; o < O; ++o)
        for (size_t i = 0; i < I; ++i) {
            size_t base = o * A * I + i;
            float sum = 0.0f;
            for (size_t k = 0; k < A; ++k) { float ds = dout[base + k * I] * s[base + k * I]; sum += ds; }
            for (size_t k = 0; k < A; ++k) {
                float diff = dout[base + k * I] - sum;
                out[base + k * I] = s[base + k * I] * diff;
            }
        }
}

void or_layernorm_bwd(const float* y, const float* var, const float* dout, const size_t* shape, int ndim, int axis, float* out) {
    /* tape.rs:1162-1186 (the correct per-row variance; not layernorm.ml:71) */
    size_t O, A, I;
    outer_axis_inner(shape, ndim, axis, &O, &A, &I);
#pragma omp parallel for num_threads(g_threads) schedule(static) collapse(2)
    for (size_t o = 0; o < O; ++o)
        for (size_t i = 0; i < I; ++i) {
            size_t base = o * A * I + i;
            float inv_sigma = 1.0f / sqrtf(var[o * I + i] + 1e-5f);
            float s1 = 0.0f, s2 = 0.0f;
            for (size_t k = 0; k < A; ++k) s1 += dout[base + k * I];
            float dy_mean = s1 / (float)A;
            for (size_t k = 0; k < A; ++k) { float dyy = dout[base + k * I] * y[base + k * I]; s2 += dyy; }
            float dyy_mean = s2 / (float)A;
            for (size_t k = 0; k < A; ++k) {
                float yv = y[base + k * I];
                float y_term = yv * dyy_mean;
                float tmp = dout[base + k * I] - dy_mean;
                float numer = tmp - y_term;
                out[base + k * I] = numer * inv_sigma;
            }
        }
}

void or_cross_entropy_bwd(const float* probs, size_t n, size_t c, const int32_t* targets, float dout0, float* out) {
    /* tape.rs:1200-1214 */
    float scale = dout0 / (float)n;
    memcpy(out, probs, n * c * sizeof(float));
    for (size_t i = 0; i < n; ++i) out[i * c + (size_t)targets[i]] -= 1.0f;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < n * c; ++i) out[i] *= scale;
}

void or_embedding_bwd(const float* dout, const int32_t* idx, size_t t, size_t dim, size_t vocab, float* out) {
    /* tensor_scatter_add, metal.rs:1665-1688: t-ordered accumulation */
    memset(out, 0, vocab * dim * sizeof(float));
    for (size_t i = 0; i < t; ++i) {
        size_t r = (size_t)idx[i];
        for (size_t d = 0; d < dim; ++d) out[r * dim + d] += dout[i * dim + d];
    }
}

/* ========================================================================
 * Optimizer — examples/nanogpt_modular.ml:97-108 ("AdamW" = Adam + L2)
 * ====================================================================== */
void or_adam_l2_update(float* p, const float* g, float* m, float* v, size_t n,
                       float lr, float b1, float b2, float eps, float wd, int64_t t) {
    float bc1 = 1.0f - powf(b1, (float)t); /* line 99, `**` = f32 powf */
    float bc2 = 1.0f - powf(b2, (float)t); /* line 100 */
    float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    for (size_t i = 0; i < n; ++i) {
        float gg = g[i] + p[i] * wd;                 /* line 103 */
        float mm = m[i] * b1 + gg * omb1;            /* line 104 */
        float vv = v[i] * b2 + (gg * omb2) * gg;     /* line 105 */
        float m_hat = mm / bc1;                      /* line 106 */
        float v_hat = vv / bc2;                      /* line 107 */
        float upd = (m_hat * lr) / (sqrtf(v_hat) + eps);
        p[i] = p[i] - upd;                           /* line 108 */
        m[i] = mm;
        v[i] = vv;
    }
}

/* ========================================================================
 * XOR — examples/xor.ml
 * ====================================================================== */
float or_xor_train(int steps, float lr, float* loss_at, float* preds_out, float* params_out) {
    const float x[8] = {0, 0, 0, 1, 1, 0, 1, 1};
    const float target[4] = {0, 1, 1, 0};
    const float ones41[4] = {1, 1, 1, 1};
    float w1[16] = {0.5f, -0.6f, 0.7f, -0.4f, 0.3f, -0.5f, 0.6f, -0.3f,
                    -0.4f, 0.5f, -0.6f, 0.7f, -0.3f, 0.4f, -0.5f, 0.6f};
    float b1[8] = {0.1f, -0.1f, 0.1f, -0.1f, 0.1f, -0.1f, 0.1f, -0.1f};
    float w2[8] = {0.6f, -0.5f, 0.4f, -0.6f, 0.5f, -0.4f, 0.6f, -0.5f};
    float b2[1] = {0.0f};
    const int report[6] = {0, 500, 1000, 2000, 5000, 9999};
    float loss = 0.0f, out[4];
    size_t s42[2] = {4, 2}, s28[2] = {2, 8}, s41[2] = {4, 1}, s18[2] = {1, 8}, s81[2] = {8, 1}, s11[2] = {1, 1};
    size_t s48[2] = {4, 8}, s14[2] = {1, 4}, s24[2] = {2, 4}, s84[2] = {8, 4};
    for (int step = 0; step < steps; ++step) {
        float t1[32], t2[32], z1[32], h[32], u1[4], u2[4], z2[4], diff[4], sq[4];
        or_matmul(x, s42, 2, w1, s28, 2, t1);          /* x @ w1 */
        or_matmul(ones41, s41, 2, b1, s18, 2, t2);     /* ones41 @ b1 */
        for (int i = 0; i < 32; ++i) z1[i] = t1[i] + t2[i];
        or_unary(OR_SIGMOID, z1, 32, h);
        or_matmul(h, s48, 2, w2, s81, 2, u1);
        or_matmul(ones41, s41, 2, b2, s11, 2, u2);
        for (int i = 0; i < 4; ++i) z2[i] = u1[i] + u2[i];
        or_unary(OR_SIGMOID, z2, 4, out);
        for (int i = 0; i < 4; ++i) { diff[i] = out[i] - target[i]; sq[i] = diff[i] * diff[i]; }
        loss = or_sum_all(sq, 4); /* __reduce_all_sum_fwd: sequential */
        for (int r = 0; r < 6; ++r) if (loss_at && step == report[r]) loss_at[r] = loss;
        float dout[4], dz2[4], hT[32], dw2[8], onesT[4], db2[1], w2T[8], dh[32], dz1[32], xT[8], dw1[16], db1[8];
        for (int i = 0; i < 4; ++i) dout[i] = 2.0f * diff[i];
        for (int i = 0; i < 4; ++i) dz2[i] = (dout[i] * out[i]) * (1.0f - out[i]); /* xor.ml:1-2 */
        size_t p10[2] = {1, 0};
        or_permute(h, s48, 2, p10, hT);
        or_matmul(hT, s84, 2, dz2, s41, 2, dw2);
        or_permute(ones41, s41, 2, p10, onesT);
        or_matmul(onesT, s14, 2, dz2, s41, 2, db2);
        or_permute(w2, s81, 2, p10, w2T);
        or_matmul(dz2, s41, 2, w2T, s18, 2, dh);
        for (int i = 0; i < 32; ++i) dz1[i] = (dh[i] * h[i]) * (1.0f - h[i]);
        or_permute(x, s42, 2, p10, xT);
        or_matmul(xT, s24, 2, dz1, s48, 2, dw1);
        or_matmul(onesT, s14, 2, dz1, s48, 2, db1);
        for (int i = 0; i < 16; ++i) w1[i] = w1[i] - dw1[i] * lr;
        for (int i = 0; i < 8; ++i) b1[i] = b1[i] - db1[i] * lr;
        for (int i = 0; i < 8; ++i) w2[i] = w2[i] - dw2[i] * lr;
        b2[0] = b2[0] - db2[0] * lr;
    }
    if (preds_out) memcpy(preds_out, out, sizeof(out));
    if (params_out) {
        memcpy(params_out, w1, sizeof(w1));
        memcpy(params_out + 16, b1, sizeof(b1));
        memcpy(params_out + 24, w2, sizeof(w2));
        params_out[32] = b2[0];
    }
    return loss;
}

/* ========================================================================
 * nanoGPT — examples/nanogpt_modular.ml:38-108 with L blocks, H heads
 * ====================================================================== */
typedef struct {
    float* d;
    int nd;
    size_t sh[8];
    size_t n;
} T;

static T tnew(int nd, const size_t* sh) {
    T t;
    memset(&t, 0, sizeof(t));
    t.nd = nd;
    t.n = 1;
    for (int i = 0; i < nd; ++i) { t.sh[i] = sh[i]; t.n *= sh[i]; }
    t.d = (float*)malloc((t.n ? t.n : 1) * sizeof(float));
    if (!t.d) die("out of host memory");
    return t;
}
static T tnew2(size_t a, size_t b) { size_t s[2] = {a, b}; return tnew(2, s); }
static T tnew3(size_t a, size_t b, size_t c) { size_t s[3] = {a, b, c}; return tnew(3, s); }
static T tnew1(size_t a) { size_t s[1] = {a}; return tnew(1, s); }
static void tfree(T* t) { free(t->d); t->d = NULL; }

/* matmul, and the two VJP forms of matmul_bwd (tape.rs:1236-1266):
 * dA = dout @ transpose(B), dB = transpose(A) @ dout, transposes materialized */
static T mm(const T* a, const T* b) {
    T o = (a->nd == 3 && b->nd == 3) ? tnew3(a->sh[0], a->sh[1], b->sh[2]) : tnew2(a->sh[0], b->sh[1]);
    or_matmul(a->d, a->sh, a->nd, b->d, b->sh, b->nd, o.d);
    return o;
}
static T transpose_last2(const T* x) {
    T o;
    if (x->nd == 2) {
        o = tnew2(x->sh[1], x->sh[0]);
        size_t p[2] = {1, 0};
        or_permute(x->d, x->sh, 2, p, o.d);
    } else {
        o = tnew3(x->sh[0], x->sh[2], x->sh[1]);
        size_t p[3] = {0, 2, 1};
        or_permute(x->d, x->sh, 3, p, o.d);
    }
    return o;
}
static T mm_bwd_a(const T* b, const T* dout) { T bt = transpose_last2(b); T r = mm(dout, &bt); tfree(&bt); return r; }
static T mm_bwd_b(const T* a, const T* dout) { T at = transpose_last2(a); T r = mm(&at, dout); tfree(&at); return r; }

static void add_into(T* acc, const T* x) { /* grad_acc = __broadcast_add_fwd(old, new) */
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < acc->n; ++i) acc->d[i] = acc->d[i] + x->d[i];
}

struct or_gpt {
    int V, Tn, C, H, L, B;
    float lr, b1, b2, eps, wd;
    int np;
    T* p;   /* params in the reference's submodule order */
    T* g;   /* grads from the last backward */
    T* m;
    T* v;
    int32_t* pos;
};

/* parameter index helpers: block l param j (0..7), then wte, wpe, ln_f, lm_head */
#define PB(l, j) ((l) * 8 + (j))
#define PT(gp, j) ((gp)->L * 8 + (j))

or_gpt* or_gpt_create(int V, int Tn, int C, int H, int L, int B, uint64_t rng_call_idx,
                      float lr, float b1, float b2, float eps, float wd) {
    or_gpt* g = (or_gpt*)calloc(1, sizeof(or_gpt));
    g->V = V; g->Tn = Tn; g->C = C; g->H = H; g->L = L; g->B = B;
    g->lr = lr; g->b1 = b1; g->b2 = b2; g->eps = eps; g->wd = wd;
    g->np = 8 * L + 4;
    g->p = (T*)calloc((size_t)g->np, sizeof(T));
    g->g = (T*)calloc((size_t)g->np, sizeof(T));
    g->m = (T*)calloc((size_t)g->np, sizeof(T));
    g->v = (T*)calloc((size_t)g->np, sizeof(T));
    size_t C4 = (size_t)4 * C;
    uint64_t call = rng_call_idx;
    /* randn(...) * init_scale with init_scale = ones(1,1) * 0.02 (make_block, lines 110-121) */
#define RANDN_INTO(tt) do { or_randn(call++, (tt).n, (tt).d); for (size_t q_ = 0; q_ < (tt).n; ++q_) (tt).d[q_] = (tt).d[q_] * 0.02f; } while (0)
#define ONES_INTO(tt) do { for (size_t q_ = 0; q_ < (tt).n; ++q_) (tt).d[q_] = 1.0f; } while (0)
    for (int l = 0; l < L; ++l) {
        g->p[PB(l, 0)] = tnew1((size_t)C); ONES_INTO(g->p[PB(l, 0)]);
        for (int j = 1; j <= 4; ++j) { g->p[PB(l, j)] = tnew2((size_t)C, (size_t)C); RANDN_INTO(g->p[PB(l, j)]); }
        g->p[PB(l, 5)] = tnew1((size_t)C); ONES_INTO(g->p[PB(l, 5)]);
        g->p[PB(l, 6)] = tnew2((size_t)C, C4); RANDN_INTO(g->p[PB(l, 6)]);
        g->p[PB(l, 7)] = tnew2(C4, (size_t)C); RANDN_INTO(g->p[PB(l, 7)]);
    }
    /* GPT params (nanogpt_modular.ml:155-160): wte, wpe, ln_f, lm_head */
    g->p[PT(g, 0)] = tnew2((size_t)V, (size_t)C); RANDN_INTO(g->p[PT(g, 0)]);
    g->p[PT(g, 1)] = tnew2((size_t)Tn, (size_t)C); RANDN_INTO(g->p[PT(g, 1)]);
    g->p[PT(g, 2)] = tnew1((size_t)C); ONES_INTO(g->p[PT(g, 2)]);
    g->p[PT(g, 3)] = tnew2((size_t)C, (size_t)V); RANDN_INTO(g->p[PT(g, 3)]);
#undef RANDN_INTO
#undef ONES_INTO
    for (int i = 0; i < g->np; ++i) {
        g->m[i] = tnew(g->p[i].nd, g->p[i].sh);
        g->v[i] = tnew(g->p[i].nd, g->p[i].sh);
        memset(g->m[i].d, 0, g->m[i].n * sizeof(float));
        memset(g->v[i].d, 0, g->v[i].n * sizeof(float));
        g->g[i].d = NULL;
    }
    g->pos = (int32_t*)malloc((size_t)B * Tn * sizeof(int32_t));
    for (int b = 0; b < B; ++b) for (int t = 0; t < Tn; ++t) g->pos[b * Tn + t] = t; /* lines 80-84 */
    return g;
}

void or_gpt_free(or_gpt* g) {
    if (!g) return;
    for (int i = 0; i < g->np; ++i) { tfree(&g->p[i]); tfree(&g->g[i]); tfree(&g->m[i]); tfree(&g->v[i]); }
    free(g->p); free(g->g); free(g->m); free(g->v); free(g->pos); free(g);
}
int or_gpt_nparams(const or_gpt* g) { return g->np; }
size_t or_gpt_param_len(const or_gpt* g, int i) { return g->p[i].n; }
void or_gpt_get_param(const or_gpt* g, int i, float* out) { memcpy(out, g->p[i].d, g->p[i].n * sizeof(float)); }
void or_gpt_set_param(or_gpt* g, int i, const float* in) { memcpy(g->p[i].d, in, g->p[i].n * sizeof(float)); }
void or_gpt_get_moment(const or_gpt* g, int i, int which, float* out) {
    memcpy(out, (which ? g->v : g->m)[i].d, g->p[i].n * sizeof(float));
}
void or_gpt_set_moment(or_gpt* g, int i, int which, const float* in) {
    memcpy((which ? g->v : g->m)[i].d, in, g->p[i].n * sizeof(float));
}
void or_gpt_get_grad(const or_gpt* g, int i, float* out) {
    if (g->g[i].d) memcpy(out, g->g[i].d, g->g[i].n * sizeof(float));
    else memset(out, 0, g->p[i].n * sizeof(float));
}

/* head fold [N,C] -> [B,T,H,hs] -> permute(0,2,1,3) -> [B*H,T,hs] (lines 51-53) */
static T head_fold(const T* x, int B, int Tn, int H, int hs) {
    size_t sh4[4] = {(size_t)B, (size_t)Tn, (size_t)H, (size_t)hs};
    size_t p[4] = {0, 2, 1, 3};
    T o = tnew3((size_t)B * H, (size_t)Tn, (size_t)hs);
    or_permute(x->d, sh4, 4, p, o.d);
    return o;
}
/* head unfold [B*H,T,hs] -> [B,H,T,hs] -> permute(0,2,1,3) -> [N,C] (line 62) */
static T head_unfold(const T* x, int B, int Tn, int H, int hs) {
    size_t sh4[4] = {(size_t)B, (size_t)H, (size_t)Tn, (size_t)hs};
    size_t p[4] = {0, 2, 1, 3};
    T o = tnew2((size_t)B * Tn, (size_t)H * hs);
    or_permute(x->d, sh4, 4, p, o.d);
    return o;
}

typedef struct {
    T x, y1, var1, xn1, Q, K, V, Kt, P, att_out, x2, y2, var2, xn2, h, ge;
} BlockCache;

static void ln_fwd(const T* x, T* y, T* var) {
    *y = tnew(x->nd, x->sh);
    *var = tnew2(x->sh[0], 1);
    or_layernorm_axis(x->d, x->sh, 2, 1, y->d, var->d);
}
static T mul_row(const T* y, const T* w) { /* [N,C] * [C] broadcast */
    T o = tnew(y->nd, y->sh);
    size_t C = y->sh[1];
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < y->n; ++i) o.d[i] = y->d[i] * w->d[i % C];
    return o;
}
/* mul VJP for y * w with w [C]: dy = dout * w; dw = sum_to_shape(y * dout) */
static void mul_row_bwd(const T* y, const T* w, const T* dout, T* dy, T* dw) {
    size_t C = y->sh[1];
    *dy = tnew(y->nd, y->sh);
    T full = tnew(y->nd, y->sh);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < y->n; ++i) { dy->d[i] = dout->d[i] * w->d[i % C]; full.d[i] = y->d[i] * dout->d[i]; }
    *dw = tnew1(C);
    size_t tsh[1] = {C};
    or_sum_to_shape(full.d, y->sh, 2, tsh, 1, dw->d);
    tfree(&full);
}
static T ln_bwd(const T* y, const T* var, const T* dout) {
    T o = tnew(y->nd, y->sh);
    or_layernorm_bwd(y->d, var->d, dout->d, y->sh, 2, 1, o.d);
    return o;
}
static void free_cache(BlockCache* c) {
    tfree(&c->y1); tfree(&c->var1); tfree(&c->xn1); tfree(&c->Q); tfree(&c->K); tfree(&c->V);
    tfree(&c->Kt); tfree(&c->P); tfree(&c->att_out); tfree(&c->x2); tfree(&c->y2); tfree(&c->var2);
    tfree(&c->xn2); tfree(&c->h); tfree(&c->ge);
}

float or_gpt_loss_and_grads(or_gpt* g, const int32_t* xt, const int32_t* yt, float* logits_out) {
    const int B = g->B, Tn = g->Tn, C = g->C, H = g->H, L = g->L, V = g->V;
    const int hs = C / H;
    const size_t N = (size_t)B * Tn;
    const float scale = 1.0f / sqrtf((float)hs);
    /* forward (nanogpt_modular.ml:75-91, 38-68) */
    T te = tnew2(N, (size_t)C), pe = tnew2(N, (size_t)C);
    or_embedding(g->p[PT(g, 0)].d, (size_t)V, (size_t)C, xt, N, te.d);
    or_embedding(g->p[PT(g, 1)].d, (size_t)Tn, (size_t)C, g->pos, N, pe.d);
    T x = tnew2(N, (size_t)C);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < x.n; ++i) x.d[i] = te.d[i] + pe.d[i];
    tfree(&te); tfree(&pe);
    BlockCache* cache = (BlockCache*)calloc((size_t)L, sizeof(BlockCache));
    T mask = tnew2((size_t)Tn, (size_t)Tn);
    or_causal_mask((size_t)Tn, mask.d);
    for (int l = 0; l < L; ++l) {
        BlockCache* c = &cache[l];
        c->x = x;
        ln_fwd(&x, &c->y1, &c->var1);
        c->xn1 = mul_row(&c->y1, &g->p[PB(l, 0)]);
        T q = mm(&c->xn1, &g->p[PB(l, 1)]);
        c->Q = head_fold(&q, B, Tn, H, hs); tfree(&q);
        T k = mm(&c->xn1, &g->p[PB(l, 2)]);
        c->K = head_fold(&k, B, Tn, H, hs); tfree(&k);
        T v = mm(&c->xn1, &g->p[PB(l, 3)]);
        c->V = head_fold(&v, B, Tn, H, hs); tfree(&v);
        c->Kt = transpose_last2(&c->K);
        T S = mm(&c->Q, &c->Kt);
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < S.n; ++i) S.d[i] = S.d[i] * scale;                 /* scores * scale */
        size_t TT = (size_t)Tn * Tn;
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < S.n; ++i) S.d[i] = S.d[i] + mask.d[i % TT];       /* + vmask */
        c->P = tnew(S.nd, S.sh);
        or_softmax_axis(S.d, S.sh, 3, 2, c->P.d);
        tfree(&S);
        T ao = mm(&c->P, &c->V);
        c->att_out = head_unfold(&ao, B, Tn, H, hs); tfree(&ao);
        T proj = mm(&c->att_out, &g->p[PB(l, 4)]);
        c->x2 = tnew2(N, (size_t)C);
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < proj.n; ++i) c->x2.d[i] = x.d[i] + proj.d[i];
        tfree(&proj);
        ln_fwd(&c->x2, &c->y2, &c->var2);
        c->xn2 = mul_row(&c->y2, &g->p[PB(l, 5)]);
        c->h = mm(&c->xn2, &g->p[PB(l, 6)]);
        c->ge = tnew(c->h.nd, c->h.sh);
        or_unary(OR_GELU, c->h.d, c->h.n, c->ge.d);
        T mo = mm(&c->ge, &g->p[PB(l, 7)]);
        T xn = tnew2(N, (size_t)C);
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < xn.n; ++i) xn.d[i] = c->x2.d[i] + mo.d[i];
        tfree(&mo);
        x = xn;
    }
    tfree(&mask);
    T yf, varf;
    ln_fwd(&x, &yf, &varf);
    T xf = mul_row(&yf, &g->p[PT(g, 2)]);
    T logits = mm(&xf, &g->p[PT(g, 3)]);
    if (logits_out) memcpy(logits_out, logits.d, logits.n * sizeof(float));
    T probs = tnew(logits.nd, logits.sh);
    float loss = or_cross_entropy(logits.d, N, (size_t)V, yt, probs.d);
    tfree(&logits);

    /* backward: reverse of the tape records (tape.rs:458-691) */
    for (int i = 0; i < g->np; ++i) tfree(&g->g[i]);
    T dlogits = tnew(probs.nd, probs.sh);
    or_cross_entropy_bwd(probs.d, N, (size_t)V, yt, 1.0f, dlogits.d); /* seed ones_like(loss) */
    tfree(&probs);
    g->g[PT(g, 3)] = mm_bwd_b(&xf, &dlogits);
    T dxf = mm_bwd_a(&g->p[PT(g, 3)], &dlogits);
    tfree(&dlogits);
    T dyf, dlnf;
    mul_row_bwd(&yf, &g->p[PT(g, 2)], &dxf, &dyf, &dlnf);
    g->g[PT(g, 2)] = dlnf;
    tfree(&dxf);
    T dx = ln_bwd(&yf, &varf, &dyf);
    tfree(&dyf); tfree(&yf); tfree(&varf); tfree(&xf);
    tfree(&x); /* output of the last block */
    for (int l = L - 1; l >= 0; --l) {
        BlockCache* c = &cache[l];
        /* x_next = x2 + mo: dx2 = dx (first contribution), dmo = dx */
        T dx2 = tnew(dx.nd, dx.sh);
        memcpy(dx2.d, dx.d, dx.n * sizeof(float));
        g->g[PB(l, 7)] = mm_bwd_b(&c->ge, &dx);
        T dge = mm_bwd_a(&g->p[PB(l, 7)], &dx);
        tfree(&dx);
        T dh = tnew(c->h.nd, c->h.sh);
        or_unary_bwd(OR_GELU, c->h.d, dge.d, c->h.n, dh.d);
        tfree(&dge);
        g->g[PB(l, 6)] = mm_bwd_b(&c->xn2, &dh);
        T dxn2 = mm_bwd_a(&g->p[PB(l, 6)], &dh);
        tfree(&dh);
        T dy2, dln2;
        mul_row_bwd(&c->y2, &g->p[PB(l, 5)], &dxn2, &dy2, &dln2);
        g->g[PB(l, 5)] = dln2;
        tfree(&dxn2);
        T dx2_ln = ln_bwd(&c->y2, &c->var2, &dy2);
        tfree(&dy2);
        add_into(&dx2, &dx2_ln); /* grads[x2] = old + new */
        tfree(&dx2_ln);
        /* x2 = x + proj */
        T dxb = tnew(dx2.nd, dx2.sh);
        memcpy(dxb.d, dx2.d, dx2.n * sizeof(float));
        g->g[PB(l, 4)] = mm_bwd_b(&c->att_out, &dx2);
        T datt = mm_bwd_a(&g->p[PB(l, 4)], &dx2);
        tfree(&dx2);
        /* unfold backward: reshape -> permute(0,2,1,3) -> reshape */
        T dao = head_fold(&datt, B, Tn, H, hs);
        tfree(&datt);
        /* ao = P @ V */
        T dP = mm_bwd_a(&c->V, &dao);
        T dV = mm_bwd_b(&c->P, &dao);
        tfree(&dao);
        T dS = tnew(dP.nd, dP.sh);
        or_softmax_bwd(c->P.d, dP.d, dP.sh, 3, 2, dS.d);
        tfree(&dP);
        /* masked = scores + vmask: dscores = dS; scores = QKt * scale: dQKt = dS * scale */
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < dS.n; ++i) dS.d[i] = dS.d[i] * scale;
        T dQ = mm_bwd_a(&c->Kt, &dS);
        T dKt = mm_bwd_b(&c->Q, &dS);
        tfree(&dS);
        T dK = transpose_last2(&dKt);
        tfree(&dKt);
        /* V chain, then K chain, then Q chain (reverse record order) */
        T dv = head_unfold(&dV, B, Tn, H, hs); tfree(&dV);
        g->g[PB(l, 3)] = mm_bwd_b(&c->xn1, &dv);
        T dxn1 = mm_bwd_a(&g->p[PB(l, 3)], &dv);
        tfree(&dv);
        T dk = head_unfold(&dK, B, Tn, H, hs); tfree(&dK);
        g->g[PB(l, 2)] = mm_bwd_b(&c->xn1, &dk);
        T dxk = mm_bwd_a(&g->p[PB(l, 2)], &dk);
        tfree(&dk);
        add_into(&dxn1, &dxk); tfree(&dxk);
        T dq = head_unfold(&dQ, B, Tn, H, hs); tfree(&dQ);
        g->g[PB(l, 1)] = mm_bwd_b(&c->xn1, &dq);
        T dxq = mm_bwd_a(&g->p[PB(l, 1)], &dq);
        tfree(&dq);
        add_into(&dxn1, &dxq); tfree(&dxq);
        T dy1, dln1;
        mul_row_bwd(&c->y1, &g->p[PB(l, 0)], &dxn1, &dy1, &dln1);
        g->g[PB(l, 0)] = dln1;
        tfree(&dxn1);
        T dx_ln = ln_bwd(&c->y1, &c->var1, &dy1);
        tfree(&dy1);
        add_into(&dxb, &dx_ln); /* grads[x] = (from x2 add) + (from LN) */
        tfree(&dx_ln);
        tfree(&c->x); /* block input (x0 for l == 0, else the previous block's output) */
        free_cache(c);
        dx = dxb;
    }
    /* x0 = te + pe */
    g->g[PT(g, 0)] = tnew2((size_t)V, (size_t)C);
    or_embedding_bwd(dx.d, xt, N, (size_t)C, (size_t)V, g->g[PT(g, 0)].d);
    g->g[PT(g, 1)] = tnew2((size_t)Tn, (size_t)C);
    or_embedding_bwd(dx.d, g->pos, N, (size_t)C, (size_t)Tn, g->g[PT(g, 1)].d);
    tfree(&dx);
    free(cache);
    return loss;
}

float or_gpt_step(or_gpt* g, const int32_t* x, const int32_t* y, int64_t t) {
    float loss = or_gpt_loss_and_grads(g, x, y, NULL);
    for (int i = 0; i < g->np; ++i)
        or_adam_l2_update(g->p[i].d, g->g[i].d, g->m[i].d, g->v[i].d, g->p[i].n,
                          g->lr, g->b1, g->b2, g->eps, g->wd, t);
    return loss;
}
