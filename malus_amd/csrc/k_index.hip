// Index kernels: embedding gather, its deterministic scatter-add VJP, and
// permute.  Integer index work is exact; the scatter-add sums each weight
// row's contributions in increasing token order, the order the reference
// accumulates them (transformer_bwd.ml:83-91, metal.rs:1665-1688), so it is
// bit-identical to the host loop.
#include "common.h"

namespace malus {
namespace k {
namespace {

// embedding.ml:11-16: out[t, c] = w[idx[t], c].  One wave per token row,
// float4 over the embedding dim when it is a multiple of 4.
__global__ __launch_bounds__(256) void k_embedding(const float* __restrict__ w, const int32_t* __restrict__ idx,
                                                   float* __restrict__ out, size_t t, uint32_t v, uint32_t d,
                                                   int32_t* __restrict__ err) {
  const size_t row = (size_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= t) return;
  const int32_t r = idx[row];
  float* o = out + row * d;
  if (r < 0 || (uint32_t)r >= v) {  // out of range: zero row, flag for the next flush
    for (uint32_t c = lane; c < d; c += 64) o[c] = 0.0f;
    if (lane == 0) *err = 1;
    return;
  }
  const float* src = w + (size_t)r * d;
  if ((d & 3) == 0) {
    for (uint32_t c = lane; c < d / 4; c += 64)
      reinterpret_cast<float4*>(o)[c] = reinterpret_cast<const float4*>(src)[c];
  } else {
    for (uint32_t c = lane; c < d; c += 64) o[c] = src[c];
  }
}

// Scatter-add, step 1: block per vocab row v counts its tokens.
__global__ __launch_bounds__(256) void k_emb_count(const int32_t* __restrict__ idx, size_t t, uint32_t* __restrict__ count) {
  __shared__ uint32_t part[4];
  const uint32_t v = blockIdx.x;
  uint32_t c = 0;
  for (size_t i = threadIdx.x; i < t; i += blockDim.x) c += (idx[i] == (int32_t)v) ? 1u : 0u;
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = c;
  __syncthreads();
  if (threadIdx.x == 0) count[v] = part[0] + part[1] + part[2] + part[3];
}

// step 2: exclusive scan of counts (single block, V small).
__global__ void k_emb_scan(const uint32_t* __restrict__ count, uint32_t* __restrict__ offs, uint32_t v) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    uint32_t s = 0;
    for (uint32_t i = 0; i < v; ++i) { offs[i] = s; s += count[i]; }
    offs[v] = s;
  }
}

// step 3: block per vocab row v writes its token positions in increasing
// order (a block-wide ordered compaction over 256-token windows).
__global__ __launch_bounds__(256) void k_emb_place(const int32_t* __restrict__ idx, size_t t,
                                                   const uint32_t* __restrict__ offs, uint32_t* __restrict__ pos) {
  __shared__ uint32_t wave_cnt[4];
  const uint32_t v = blockIdx.x;
  uint32_t base = offs[v];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  for (size_t w0 = 0; w0 < t; w0 += blockDim.x) {
    size_t i = w0 + threadIdx.x;
    bool hit = i < t && idx[i] == (int32_t)v;
    unsigned long long mask = __ballot(hit);
    uint32_t before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = (uint32_t)__popcll(mask);
    __syncthreads();
    uint32_t wave_base = 0;
    for (int q = 0; q < wave; ++q) wave_base += wave_cnt[q];
    if (hit) pos[base + wave_base + before] = (uint32_t)i;
    uint32_t tot = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
    base += tot;
  }
}

// step 4: dw[v, c] = sum over that row's token list, in list order.
__global__ __launch_bounds__(256) void k_emb_accum(const float* __restrict__ dout, const uint32_t* __restrict__ offs,
                                                   const uint32_t* __restrict__ pos, float* __restrict__ dw, uint32_t v,
                                                   uint32_t d, uint32_t col_blocks) {
  const uint32_t row = blockIdx.x / col_blocks;
  const uint32_t c = (blockIdx.x % col_blocks) * blockDim.x + threadIdx.x;
  if (row >= v || c >= d) return;
  const uint32_t beg = offs[row], end = offs[row + 1];
  float acc = 0.0f;
  uint32_t k = beg;
  // independent loads issued ahead, the adds stay in list order
  for (; k + 4 <= end; k += 4) {
    float a0 = dout[(size_t)pos[k] * d + c];
    float a1 = dout[(size_t)pos[k + 1] * d + c];
    float a2 = dout[(size_t)pos[k + 2] * d + c];
    float a3 = dout[(size_t)pos[k + 3] * d + c];
    acc += a0; acc += a1; acc += a2; acc += a3;
  }
  for (; k < end; ++k) acc += dout[(size_t)pos[k] * d + c];
  dw[(size_t)row * d + c] = acc;
}

// Two-launch form for small vocabularies (v * t list slots fit the pool).
// k_emb_list: block per vocab row v writes the positions of its tokens, in
// increasing order, at pos[v * t ..] and their count.  Thread i owns the
// contiguous tokens [i * per, (i + 1) * per) (per a multiple of 4, read as
// int4 with VEC); a block exclusive scan of the per-thread hit counts
// (thread order = token order) places them.
template <bool VEC>
__global__ __launch_bounds__(256) void k_emb_list(const int32_t* __restrict__ idx, size_t t, uint32_t* __restrict__ pos,
                                                  uint32_t* __restrict__ count) {
  __shared__ uint32_t wave_tot[4];
  const int32_t v = (int32_t)blockIdx.x;
  const size_t per = ((t + 255) / 256 + 3) / 4 * 4;
  const size_t beg = min(t, (size_t)threadIdx.x * per), end = min(t, beg + per);
  const int4* idx4 = reinterpret_cast<const int4*>(idx);
  uint32_t c = 0;
  if (VEC) {  // t % 4 == 0, so [beg, end) is whole int4s
#pragma unroll 4
    for (size_t q = beg / 4; q < end / 4; ++q) {
      const int4 x = idx4[q];
      c += (x.x == v ? 1u : 0u) + (x.y == v ? 1u : 0u) + (x.z == v ? 1u : 0u) + (x.w == v ? 1u : 0u);
    }
  } else {
#pragma unroll 4
    for (size_t i = beg; i < end; ++i) c += idx[i] == v ? 1u : 0u;
  }
  // inclusive scan over the wave, then over the four waves
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t inc = c;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  uint32_t base = inc - c;
  for (int q = 0; q < wave; ++q) base += wave_tot[q];
  uint32_t* out = pos + (size_t)blockIdx.x * t;
  if (c) {
    if (VEC) {
#pragma unroll 4
      for (size_t q = beg / 4; q < end / 4; ++q) {
        const int4 x = idx4[q];
        const uint32_t i = (uint32_t)(4 * q);
        if (x.x == v) out[base++] = i;
        if (x.y == v) out[base++] = i + 1;
        if (x.z == v) out[base++] = i + 2;
        if (x.w == v) out[base++] = i + 3;
      }
    } else {
      for (size_t i = beg; i < end; ++i)
        if (idx[i] == v) out[base++] = (uint32_t)i;
    }
  }
  if (threadIdx.x == 255) count[blockIdx.x] = base;
}

// k_emb_rows: dw[v, 4c .. 4c + 3] = the sum of dout[t, 4c ..] over row v's
// token list, in list order (the same adds as k_emb_accum).  One lane per
// (row, 4-column group), lanes packed across rows.  Each chain is a run of
// dependent adds over its list, so the list is walked in batches of R
// float4 loads that are all in flight before their adds, with the next
// batch's positions loaded meanwhile (a chain of ~250 tokens then costs a
// handful of memory round trips instead of one per 16 tokens).
template <int R>
__global__ __launch_bounds__(64) void k_emb_rows(const float4* __restrict__ dout, const uint32_t* __restrict__ pos,
                                                 const uint32_t* __restrict__ count, float4* __restrict__ dw, size_t t,
                                                 uint32_t d4, uint32_t chains) {
  static_assert(R % 4 == 0, "positions are loaded four at a time");
  const uint32_t g = blockIdx.x * 64 + threadIdx.x;
  if (g >= chains) return;
  const uint32_t row = g / d4, c = g % d4;
  const uint32_t n = count[row];
  const uint32_t* p = pos + (size_t)row * t;  // R > 0: 16-byte aligned (the host takes this form for t % 4 == 0)
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  uint32_t k = 0;
  if constexpr (R > 0) {
    uint4 ix[R / 4];
    if (R <= n) {
#pragma unroll
      for (int u = 0; u < R / 4; ++u) ix[u] = reinterpret_cast<const uint4*>(p)[u];
    }
    for (; k + R <= n; k += R) {
      float4 a[R];
#pragma unroll
      for (int u = 0; u < R / 4; ++u) {
        a[4 * u] = dout[(size_t)ix[u].x * d4 + c];
        a[4 * u + 1] = dout[(size_t)ix[u].y * d4 + c];
        a[4 * u + 2] = dout[(size_t)ix[u].z * d4 + c];
        a[4 * u + 3] = dout[(size_t)ix[u].w * d4 + c];
      }
      if (k + 2 * R <= n) {
#pragma unroll
        for (int u = 0; u < R / 4; ++u) ix[u] = reinterpret_cast<const uint4*>(p + k + R)[u];
      }
#pragma unroll
      for (int u = 0; u < R; ++u) {
        acc.x += a[u].x;
        acc.y += a[u].y;
        acc.z += a[u].z;
        acc.w += a[u].w;
      }
    }
  }
  for (; k + 8 <= n; k += 8) {
    float4 a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = dout[(size_t)p[k + u] * d4 + c];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc.x += a[u].x;
      acc.y += a[u].y;
      acc.z += a[u].z;
      acc.w += a[u].w;
    }
  }
  for (; k < n; ++k) {
    const float4 a = dout[(size_t)p[k] * d4 + c];
    acc.x += a.x;
    acc.y += a.y;
    acc.z += a.z;
    acc.w += a.w;
  }
  dw[(size_t)row * d4 + c] = acc;
}

struct PermDesc {
  int ndim;
  uint32_t out_shape[kMaxRank];
  uint64_t in_stride_for_out[kMaxRank];  // input stride of the input dim that output dim d reads
};

// Generic gather: out[flat] = x[in_flat] (permute.ml:79-100).
__global__ __launch_bounds__(256) void k_permute_generic(const float* __restrict__ x, float* __restrict__ out, size_t n,
                                                         PermDesc p) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t f = (size_t)blockIdx.x * blockDim.x + threadIdx.x; f < n; f += stride) {
    size_t rem = f, in = 0;
    for (int d = p.ndim - 1; d >= 0; --d) {
      size_t id = rem % p.out_shape[d];
      rem /= p.out_shape[d];
      in += id * p.in_stride_for_out[d];
    }
    out[f] = x[in];
  }
}

// Last dim kept in place: copy rows of `row` contiguous floats (float4).
__global__ __launch_bounds__(256) void k_permute_rows(const float4* __restrict__ x, float4* __restrict__ out,
                                                      size_t n_rows, uint32_t row4, PermDesc p) {
  // p describes the permutation of the leading ndim dims (row dim removed)
  size_t total = n_rows * row4, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t f = (size_t)blockIdx.x * blockDim.x + threadIdx.x; f < total; f += stride) {
    size_t r = f / row4, c = f % row4;
    size_t rem = r, in = 0;
    for (int d = p.ndim - 1; d >= 0; --d) {
      size_t id = rem % p.out_shape[d];
      rem /= p.out_shape[d];
      in += id * p.in_stride_for_out[d];
    }
    out[f] = x[in * row4 + c];
  }
}

// Batched transpose of the last two dims: x [B, R, C] -> out [B, C, R] via
// 64x64 LDS tiles (coalesced reads and writes).
__global__ __launch_bounds__(256) void k_transpose_last2(const float* __restrict__ x, float* __restrict__ out, uint32_t R,
                                                         uint32_t C, uint32_t tiles_r, uint32_t tiles_c) {
  __shared__ float tile[64][65];
  const uint32_t b = blockIdx.y;
  const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const float* xb = x + (size_t)b * R * C;
  float* ob = out + (size_t)b * R * C;
  const uint32_t lx = threadIdx.x % 64, ly = threadIdx.x / 64;  // 64 x 4
  for (uint32_t i = ly; i < 64; i += 4) {
    uint32_t r = tr * 64 + i, c = tc * 64 + lx;
    if (r < R && c < C) tile[i][lx] = xb[(size_t)r * C + c];
  }
  __syncthreads();
  for (uint32_t i = ly; i < 64; i += 4) {
    uint32_t c = tc * 64 + i, r = tr * 64 + lx;  // out[c][r]
    if (r < R && c < C) ob[(size_t)c * R + r] = tile[lx][i];
  }
  (void)tiles_r;
}

}  // namespace

// The token and position embeddings and their sum in one pass:
// out[t, c] = wa[ia[t], c] + wb[ib[t], c] (embedding.ml:11-16 twice, then the
// broadcast add: the same f32 add).  Out-of-range rows count as zero rows
// and set the error flag, as in k_embedding.
__global__ __launch_bounds__(256) void k_embedding2(const float* __restrict__ wa, const int32_t* __restrict__ ia,
                                                    uint32_t va, const float* __restrict__ wb,
                                                    const int32_t* __restrict__ ib, uint32_t vb,
                                                    float* __restrict__ out, size_t t, uint32_t d,
                                                    int32_t* __restrict__ err) {
  const size_t row = (size_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= t) return;
  const int32_t ra = ia[row], rb = ib[row];
  const bool oka = ra >= 0 && (uint32_t)ra < va, okb = rb >= 0 && (uint32_t)rb < vb;
  if ((!oka || !okb) && lane == 0) *err = 1;
  const float* pa = wa + (size_t)(oka ? ra : 0) * d;
  const float* pb = wb + (size_t)(okb ? rb : 0) * d;
  float* o = out + row * d;
  for (uint32_t c = lane; c < d / 4; c += 64) {
    const float4 a = oka ? reinterpret_cast<const float4*>(pa)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 b = okb ? reinterpret_cast<const float4*>(pb)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    reinterpret_cast<float4*>(o)[c] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
}

void embedding2(const float* wa, const int32_t* ia, size_t va, const float* wb, const int32_t* ib, size_t vb, float* out,
                size_t t, size_t d, int32_t* err, hipStream_t s) {
  if (!t || !d) return;
  if (d % 4) fail("malus: embedding2: row length %zu is not a multiple of 4", d);
  k_embedding2<<<(unsigned)((t + 3) / 4), 256, 0, s>>>(wa, ia, (uint32_t)va, wb, ib, (uint32_t)vb, out, t, (uint32_t)d,
                                                       err);
  MALUS_HIP(hipGetLastError());
}

void embedding(const float* w, const int32_t* idx, float* out, size_t t, size_t v, size_t d, int32_t* err, hipStream_t s) {
  if (!t || !d) return;
  k_embedding<<<(unsigned)((t + 3) / 4), 256, 0, s>>>(w, idx, out, t, (uint32_t)v, (uint32_t)d, err);
  MALUS_HIP(hipGetLastError());
}

void embedding_bwd(const float* dout, const int32_t* idx, float* dw, size_t t, size_t v, size_t d, hipStream_t s) {
  if (!v || !d) return;
  if (!t) { fill(dw, 0.0f, v * d, s); return; }
  size_t b_count, b_offs, b_pos;
  const auto aligned = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  if (d % 4 == 0 && v * t <= ((size_t)1 << 24) && v * (d / 4) < ((size_t)1 << 31) && aligned(dout) && aligned(dw)) {
    uint32_t* count = static_cast<uint32_t*>(pool_alloc(v * sizeof(uint32_t), &b_count));
    uint32_t* pos = static_cast<uint32_t*>(pool_alloc(v * t * sizeof(uint32_t), &b_pos));
    if (t % 4 == 0 && aligned(idx)) k_emb_list<true><<<(unsigned)v, 256, 0, s>>>(idx, t, pos, count);
    else k_emb_list<false><<<(unsigned)v, 256, 0, s>>>(idx, t, pos, count);
    MALUS_HIP(hipGetLastError());
    const uint32_t d4 = (uint32_t)(d / 4), chains = (uint32_t)(v * d4);
    if (t % 4 == 0)
      k_emb_rows<48><<<(chains + 63) / 64, 64, 0, s>>>(reinterpret_cast<const float4*>(dout), pos, count,
                                                        reinterpret_cast<float4*>(dw), t, d4, chains);
    else
      k_emb_rows<0><<<(chains + 63) / 64, 64, 0, s>>>(reinterpret_cast<const float4*>(dout), pos, count,
                                                       reinterpret_cast<float4*>(dw), t, d4, chains);
    MALUS_HIP(hipGetLastError());
    pool_free(count, b_count);
    pool_free(pos, b_pos);
    return;
  }
  uint32_t* count = static_cast<uint32_t*>(pool_alloc(v * sizeof(uint32_t), &b_count));
  uint32_t* offs = static_cast<uint32_t*>(pool_alloc((v + 1) * sizeof(uint32_t), &b_offs));
  uint32_t* pos = static_cast<uint32_t*>(pool_alloc(t * sizeof(uint32_t), &b_pos));
  k_emb_count<<<(unsigned)v, 256, 0, s>>>(idx, t, count);
  MALUS_HIP(hipGetLastError());
  k_emb_scan<<<1, 64, 0, s>>>(count, offs, (uint32_t)v);
  MALUS_HIP(hipGetLastError());
  k_emb_place<<<(unsigned)v, 256, 0, s>>>(idx, t, offs, pos);
  MALUS_HIP(hipGetLastError());
  uint32_t col_blocks = (uint32_t)((d + 255) / 256);
  k_emb_accum<<<(unsigned)(v * col_blocks), 256, 0, s>>>(dout, offs, pos, dw, (uint32_t)v, (uint32_t)d, col_blocks);
  MALUS_HIP(hipGetLastError());
  pool_free(count, b_count);
  pool_free(offs, b_offs);
  pool_free(pos, b_pos);
}

void permute(const float* x, float* out, int ndim, const size_t* in_shape, const size_t* perm, hipStream_t s) {
  size_t n = 1;
  for (int i = 0; i < ndim; ++i) n *= in_shape[i];
  if (!n) return;
  size_t in_stride[kMaxRank];
  in_stride[ndim - 1] = 1;
  for (int i = ndim - 2; i >= 0; --i) in_stride[i] = in_stride[i + 1] * in_shape[i + 1];
  bool identity = true;
  for (int i = 0; i < ndim; ++i) identity &= (perm[i] == (size_t)i);
  if (identity) { copy(x, out, n * sizeof(float), s); return; }
  // swap of the last two dims (batched transpose)
  if (ndim >= 2 && perm[ndim - 1] == (size_t)ndim - 2 && perm[ndim - 2] == (size_t)ndim - 1) {
    bool lead_id = true;
    for (int i = 0; i < ndim - 2; ++i) lead_id &= (perm[i] == (size_t)i);
    if (lead_id) {
      size_t R = in_shape[ndim - 2], C = in_shape[ndim - 1], B = n / (R * C);
      uint32_t tr = (uint32_t)((R + 63) / 64), tc = (uint32_t)((C + 63) / 64);
      if (B <= 65535) {
        dim3 grid(tr * tc, (unsigned)B);
        k_transpose_last2<<<grid, 256, 0, s>>>(x, out, (uint32_t)R, (uint32_t)C, tr, tc);
        MALUS_HIP(hipGetLastError());
        return;
      }
    }
  }
  PermDesc p{};
  // last dim untouched and float4-able: row copies
  if (ndim >= 2 && perm[ndim - 1] == (size_t)ndim - 1 && in_shape[ndim - 1] % 4 == 0) {
    size_t row = in_shape[ndim - 1];
    p.ndim = ndim - 1;
    for (int d = 0; d < ndim - 1; ++d) {
      p.out_shape[d] = (uint32_t)in_shape[perm[d]];
      p.in_stride_for_out[d] = in_stride[perm[d]] / row;
    }
    size_t rows = n / row;
    size_t blocks = (n / 4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_permute_rows<<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<const float4*>(x), reinterpret_cast<float4*>(out), rows,
                                                    (uint32_t)(row / 4), p);
    MALUS_HIP(hipGetLastError());
    return;
  }
  p.ndim = ndim;
  for (int d = 0; d < ndim; ++d) {
    p.out_shape[d] = (uint32_t)in_shape[perm[d]];
    p.in_stride_for_out[d] = in_stride[perm[d]];
  }
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  k_permute_generic<<<(unsigned)blocks, 256, 0, s>>>(x, out, n, p);
  MALUS_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace malus
