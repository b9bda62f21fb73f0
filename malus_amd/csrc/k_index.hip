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
// Both kernels take the rows of one or two tables (the token and position
// tables of one embedding sum share t and dout): global row r < va is row r
// of table a (idx_a, dw_a), a later one row r - va of table b.
// k_emb_list: block per global row r writes the positions of its tokens, in
// increasing order, at pos[r * t ..] and their count.  The tokens are taken
// in passes of 1024 x 16: thread i owns the 16 contiguous tokens
// [16 i, 16 i + 16) of a pass and keeps them in registers from its count to
// its writes (four int4 loads with VEC, all in flight together); a block
// exclusive scan of the per-thread hit counts (thread order = token order)
// places them.
template <bool VEC>
__global__ __launch_bounds__(1024) void k_emb_list(const int32_t* __restrict__ idx_a, uint32_t va,
                                                   const int32_t* __restrict__ idx_b, size_t t,
                                                   uint32_t* __restrict__ pos, uint32_t* __restrict__ count) {
  constexpr int kWaves = 16, kPer = 16;
  __shared__ uint32_t wave_tot[kWaves];
  const bool in_a = blockIdx.x < va;
  const int32_t* __restrict__ idx = in_a ? idx_a : idx_b;
  const int32_t v = (int32_t)(in_a ? blockIdx.x : blockIdx.x - va);
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t* out = pos + (size_t)blockIdx.x * t;
  uint32_t done = 0;  // hits in earlier passes
  for (size_t s = 0; s < t; s += (size_t)kPer * 1024) {
    const size_t beg = s + (size_t)kPer * threadIdx.x;
    int32_t x[kPer];
    if (VEC) {  // t % 4 == 0 and idx 16-byte aligned: whole int4s up to t
#pragma unroll
      for (int u = 0; u < kPer / 4; ++u) {
        int4 q = make_int4(-1, -1, -1, -1);
        if (beg + 4 * u + 4 <= t) q = reinterpret_cast<const int4*>(idx + beg)[u];
        x[4 * u] = q.x;
        x[4 * u + 1] = q.y;
        x[4 * u + 2] = q.z;
        x[4 * u + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kPer; ++u) x[u] = beg + u < t ? idx[beg + u] : -1;
    }
    uint32_t c = 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) c += x[u] == v ? 1u : 0u;
    // inclusive scan over the wave, then over the waves
    uint32_t inc = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(inc, off, 64);
      if (lane >= off) inc += o;
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    uint32_t base = done + inc - c, pass = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      base += q < wave ? wave_tot[q] : 0u;
      pass += wave_tot[q];
    }
    if (c) {
#pragma unroll
      for (int u = 0; u < kPer; ++u)
        if (x[u] == v) out[base++] = (uint32_t)(beg + u);
    }
    done += pass;
    __syncthreads();  // wave_tot is rewritten by the next pass
  }
  if (threadIdx.x == 0) count[blockIdx.x] = done;
}

// k_emb_cols: dw[v, c0 .. c0 + 32) = the sum of dout[p, c0 ..] over row v's
// token list p, in list order (the same adds as k_emb_accum).  Block
// (32-column block, global row), 256 threads.  Each sum is a chain of dependent
// adds, so the rows the list names are staged through LDS CH tokens at a
// time by all the block's threads (a token's 128-byte segment read by 8
// lanes as float4, 32 tokens per pass); lanes 0..31 of wave 0 then add the
// chunk in list order, one column each, while the next chunk's loads are in
// flight.  The list slot holds t entries, so the first chunk's positions are
// read beside the count that bounds them (entries past the count are never
// used as addresses), and each later chunk's a chunk ahead of its loads.
template <int CH>
__global__ __launch_bounds__(256) void k_emb_cols(const float* __restrict__ dout, const uint32_t* __restrict__ pos,
                                                  const uint32_t* __restrict__ count, float* __restrict__ dw_a,
                                                  uint32_t va, float* __restrict__ dw_b, size_t t, uint32_t d) {
  constexpr int kW = 32, kLoads = CH / 32;
  static_assert(CH % 32 == 0, "32 tokens per pass");
  __shared__ float4 buf[CH * kW / 4];
  const uint32_t row = blockIdx.y, c0 = blockIdx.x * kW;
  const uint32_t* p = pos + (size_t)row * t;
  const uint32_t seg = threadIdx.x % 8, tok = threadIdx.x / 8;
  const bool col_ok = c0 + 4 * seg < d;  // d % 4 == 0: a float4 is wholly in or out
  const float4* src = reinterpret_cast<const float4*>(dout + c0) + seg;
  const size_t d4 = d / 4;
  uint32_t pn[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) pn[j] = tok + 32 * j < t ? p[tok + 32 * j] : 0u;
  const uint32_t n = count[row];
  float4 r[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    r[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (col_ok && tok + 32 * j < n) r[j] = src[(size_t)pn[j] * d4];
  }
#pragma unroll
  for (int j = 0; j < kLoads; ++j) pn[j] = CH + tok + 32 * j < n ? p[CH + tok + 32 * j] : 0u;
  float acc = 0.0f;
  const float* lds = reinterpret_cast<const float*>(buf) + threadIdx.x;  // wave 0: lane = column
  for (uint32_t k = 0; k < n; k += CH) {
    const uint32_t m = min((uint32_t)CH, n - k);
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      if (tok + 32 * j < m) buf[(tok + 32 * j) * (kW / 4) + seg] = r[j];
    __syncthreads();
    if (k + CH < n) {  // chunk k + CH's loads (positions in pn), then chunk k + 2 CH's positions
#pragma unroll
      for (int j = 0; j < kLoads; ++j)
        if (col_ok && k + CH + tok + 32 * j < n) r[j] = src[(size_t)pn[j] * d4];
#pragma unroll
      for (int j = 0; j < kLoads; ++j) {
        const uint32_t i = k + 2 * CH + tok + 32 * j;
        pn[j] = i < n ? p[i] : 0u;
      }
    }
    if (threadIdx.x < kW) {
#pragma unroll 16
      for (uint32_t i = 0; i < m; ++i) acc += lds[i * kW];
    }
    __syncthreads();  // the chunk is read before the next one is stored
  }
  float* __restrict__ dw = row < va ? dw_a + (size_t)row * d : dw_b + (size_t)(row - va) * d;
  if (threadIdx.x < kW && c0 + threadIdx.x < d) dw[c0 + threadIdx.x] = acc;
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

namespace {
bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

// Whether rows of width d (t tokens, v rows in all) take the list-and-stage
// form.
bool emb_lists_fit(size_t t, size_t v, size_t d, const float* dout) {
  return d % 4 == 0 && v * t <= ((size_t)1 << 24) && v <= 65535 && d < ((size_t)1 << 31) && aligned16(dout);
}

// The list-and-stage form over va rows of table a and vb of table b (vb = 0:
// one table); the caller has checked emb_lists_fit for va + vb rows.
void emb_lists_and_sums(const float* dout, const int32_t* idx_a, float* dw_a, size_t va, const int32_t* idx_b,
                        float* dw_b, size_t vb, size_t t, size_t d, hipStream_t s) {
  const size_t v = va + vb;
  size_t b_count, b_pos;
  uint32_t* count = static_cast<uint32_t*>(pool_alloc(v * sizeof(uint32_t), &b_count));
  uint32_t* pos = static_cast<uint32_t*>(pool_alloc(v * t * sizeof(uint32_t), &b_pos));
  if (t % 4 == 0 && aligned16(idx_a) && aligned16(idx_b))
    k_emb_list<true><<<(unsigned)v, 1024, 0, s>>>(idx_a, (uint32_t)va, idx_b, t, pos, count);
  else
    k_emb_list<false><<<(unsigned)v, 1024, 0, s>>>(idx_a, (uint32_t)va, idx_b, t, pos, count);
  MALUS_HIP(hipGetLastError());
  // chunk size from the mean list length: one chunk for most rows
  const dim3 grid((unsigned)((d + 31) / 32), (unsigned)v);
  const size_t mean = t * (vb ? 2 : 1) / v;
  if (mean > 128) k_emb_cols<256><<<grid, 256, 0, s>>>(dout, pos, count, dw_a, (uint32_t)va, dw_b, t, (uint32_t)d);
  else if (mean > 64) k_emb_cols<128><<<grid, 256, 0, s>>>(dout, pos, count, dw_a, (uint32_t)va, dw_b, t, (uint32_t)d);
  else k_emb_cols<64><<<grid, 256, 0, s>>>(dout, pos, count, dw_a, (uint32_t)va, dw_b, t, (uint32_t)d);
  MALUS_HIP(hipGetLastError());
  pool_free(count, b_count);
  pool_free(pos, b_pos);
}
}  // namespace

bool embedding_bwd2(const float* dout, const int32_t* idx_a, float* dw_a, size_t va, const int32_t* idx_b,
                    float* dw_b, size_t vb, size_t t, size_t d, hipStream_t s) {
  if (!t || !d || !va || !vb || !emb_lists_fit(t, va + vb, d, dout) || !aligned16(dw_a) || !aligned16(dw_b))
    return false;
  emb_lists_and_sums(dout, idx_a, dw_a, va, idx_b, dw_b, vb, t, d, s);
  return true;
}

void embedding_bwd(const float* dout, const int32_t* idx, float* dw, size_t t, size_t v, size_t d, hipStream_t s) {
  if (!v || !d) return;
  if (!t) { fill(dw, 0.0f, v * d, s); return; }
  if (emb_lists_fit(t, v, d, dout) && aligned16(dw)) {
    emb_lists_and_sums(dout, idx, dw, v, idx, dw, 0, t, d, s);
    return;
  }
  size_t b_count, b_offs, b_pos;
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
