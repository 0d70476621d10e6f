// Cocktail-party head on gfx950: first-[MASK] context vector, span-interior
// means and their scores (model.py:263-298), forward and backward.
//
// The reference builds h_spans with a Python double loop over rows and over
// the zipped [SPAN] / [ES] position lists, taking x_embed[i, st+1:ed].mean(0)
// when st + 1 < ed (model.py:287-293), and scores each span by its dot
// product with the hidden state at the row's first [MASK] (:264-270, :296).
// Here one workgroup per row finds the positions (block scans give the j-th
// [SPAN] and the j-th [ES] of the row); one workgroup per (row, span, 256
// columns) sums the interior in fp32 (eight waves over interleaved rows,
// combined in a fixed order) and k_span_score dots the means with the context
// vector.  The backward spreads d score over the interior rows and the [MASK]
// row in a fixed order (one wave per row), so the results are deterministic.
#include "kd_internal.h"

namespace kd {

namespace {

constexpr int TOK_MASK = 2, TOK_SPAN = 3, TOK_ES = 4;  // data_builder.py:44-52

KD_DEV int64_t token_at(const kd_span_args& a, int b, int t) {
  const int64_t off = int64_t(b) * a.tokens_strides[0] + int64_t(t) * a.tokens_strides[1];
  return a.tokens_dtype == KD_I64 ? static_cast<const int64_t*>(a.tokens)[off]
                                  : int64_t(static_cast<const int32_t*>(a.tokens)[off]);
}

template <class E>
KD_DEV float h_at(const kd_span_args& a, int b, int t, int d) {
  const uint16_t* p = static_cast<const uint16_t*>(a.h) + int64_t(b) * a.h_strides[0] + int64_t(t) * a.h_strides[1] + d;
  return to_f32<E>(*p);
}

// One workgroup (1024 threads) per row: positions of the j-th [SPAN] and the
// j-th [ES], then the interiors [lo, hi) of the zipped pairs and the first [MASK].
__global__ __launch_bounds__(1024) void k_span_find(kd_span_args a) {
  extern __shared__ int s_pos[];  // [0, n): j-th [SPAN] position, [n, 2n): j-th [ES] position
  __shared__ int s_warp[16];
  __shared__ int s_mask;
  const int b = blockIdx.x, n = a.n_spans, T = a.T;
  for (int j = threadIdx.x; j < 2 * n; j += blockDim.x) s_pos[j] = -1;
  if (threadIdx.x == 0) s_mask = T;
  __syncthreads();
  // contiguous chunk of positions per thread, so ordinals follow position order
  const int per = (T + blockDim.x - 1) / blockDim.x;
  const int t0 = threadIdx.x * per, t1 = min(T, t0 + per);
  int ns = 0, ne = 0, first_mask = T;
  for (int t = t0; t < t1; ++t) {
    const int64_t tok = token_at(a, b, t);
    ns += tok == TOK_SPAN;
    ne += tok == TOK_ES;
    if (tok == TOK_MASK && first_mask == T) first_mask = t;
  }
  const int js = block_scan(ns, s_warp) - ns;  // exclusive: ordinal of this chunk's first [SPAN]
  const int je = block_scan(ne, s_warp) - ne;
  if (first_mask < T) atomicMin(&s_mask, first_mask);
  int cs = js, ce = je;
  for (int t = t0; t < t1; ++t) {
    const int64_t tok = token_at(a, b, t);
    if (tok == TOK_SPAN) {
      if (cs < n) s_pos[cs] = t;  // spans past n_spans are dropped
      ++cs;
    } else if (tok == TOK_ES) {
      if (ce < n) s_pos[n + ce] = t;
      ++ce;
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const int st = s_pos[j], ed = s_pos[n + j];
    const bool ok = st >= 0 && ed >= 0 && st + 1 < ed;  // zip pairs only; `if st + 1 < ed` (model.py:292)
    a.span_lo[int64_t(b) * n + j] = ok ? st + 1 : 0;
    a.span_hi[int64_t(b) * n + j] = ok ? ed : 0;
  }
  if (threadIdx.x == 0) a.mask_pos[b] = s_mask < T ? s_mask : -1;
}

// Fixed-order block sum (256 threads) of one float per thread.
KD_DEV float block_sum256(float v, float* s_red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  const float r = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  __syncthreads();
  return r;
}

// grid (n_spans + 1, B, ceil(D / 256)): block (j < n, b, c) averages span j's
// interior over the columns [256 c, 256 c + 256); block (n, b, c) copies
// those columns of h_ctx.  Wave w of 8 sums the rows lo + w, lo + w + 8, ...
// (lane l: columns 256 c + l + 64 k, k < 4) and the eight partials combine in
// a fixed order, ((w0 + w1) + (w2 + w3)) + ((w4 + w5) + (w6 + w7)).
template <class E>
__global__ __launch_bounds__(512) void k_span_pool(kd_span_args a) {
  __shared__ float s_part[8][256];
  const int j = blockIdx.x, b = blockIdx.y, n = a.n_spans, D = a.D, d0 = blockIdx.z * 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (j == n) {
    const int mp = a.mask_pos[b];
    const int d = d0 + int(threadIdx.x);
    if (threadIdx.x < 256 && d < D) a.h_ctx[int64_t(b) * D + d] = mp >= 0 ? h_at<E>(a, b, mp, d) : 0.f;
    return;
  }
  const int lo = a.span_lo[int64_t(b) * n + j], hi = a.span_hi[int64_t(b) * n + j];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int t = lo + wave; t < hi; t += 8) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = d0 + lane + 64 * k;
      if (d < D) acc[k] += h_at<E>(a, b, t, d);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) s_part[wave][lane + 64 * k] = acc[k];
  __syncthreads();
  const int d = d0 + int(threadIdx.x);
  if (threadIdx.x < 256 && d < D) {
    const int i = threadIdx.x;
    const float sum = ((s_part[0][i] + s_part[1][i]) + (s_part[2][i] + s_part[3][i])) +
                      ((s_part[4][i] + s_part[5][i]) + (s_part[6][i] + s_part[7][i]));
    a.h_spans[(int64_t(b) * n + j) * D + d] = hi > lo ? sum / float(hi - lo) : 0.f;
  }
}

// grid (n_spans, B): score of span j = sum_d h_span_j[d] h_ctx[d], thread i
// over d = i + 256 k in ascending k, then a fixed-order block sum.
__global__ __launch_bounds__(256) void k_span_score(kd_span_args a) {
  __shared__ float s_red[4];
  const int j = blockIdx.x, b = blockIdx.y, n = a.n_spans, D = a.D;
  const float* hs = a.h_spans + (int64_t(b) * n + j) * D;
  const float* hc = a.h_ctx + int64_t(b) * D;
  float part = 0.f;
  for (int d = threadIdx.x; d < D; d += 256) part = __builtin_fmaf(hs[d], hc[d], part);
  const float s = block_sum256(part, s_red);
  if (threadIdx.x == 0) a.scores[int64_t(b) * n + j] = s;
}

// grid (ceil(T / 4), B), one wave per row t of dh, written in full:
//   dh[t] = sum_{j: lo_j <= t < hi_j} ds_j h_ctx / (hi_j - lo_j)   (ascending j)
//         + [t == mask] sum_j ds_j h_span_j                          (ascending j)
// Columns go in groups of 512, lane l holding d0 + l + 64 k (k < 8).  The
// spans containing t are found 64 at a time by a wave ballot over j and added
// in ascending j; a row in no span (most rows) is written as zeros.
template <class E>
__global__ __launch_bounds__(256) void k_span_bwd(kd_span_args a) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.y, t = blockIdx.x * 4 + (threadIdx.x >> 6), n = a.n_spans, D = a.D;
  if (t >= a.T) return;
  const int mp = a.mask_pos[b];
  const int32_t* lo = a.span_lo + int64_t(b) * n;
  const int32_t* hi = a.span_hi + int64_t(b) * n;
  const float* ds = a.dscores + int64_t(b) * n;
  uint16_t* out = static_cast<uint16_t*>(a.dh) + int64_t(b) * a.dh_strides[0] + int64_t(t) * a.dh_strides[1];
  for (int d0 = 0; d0 < D; d0 += 512) {
    float c[8], g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int d = d0 + lane + 64 * k;
      c[k] = d < D ? a.h_ctx[int64_t(b) * D + d] : 0.f;
      g[k] = 0.f;
    }
    for (int j0 = 0; j0 < n; j0 += 64) {
      const int jl = j0 + lane;
      const bool in = jl < n && lo[jl] <= t && t < hi[jl];
      for (uint64_t m = __builtin_amdgcn_ballot_w64(in); m; m &= m - 1) {
        const int j = j0 + __builtin_ctzll(m);
        const float dsj = ds[j], len = float(hi[j] - lo[j]);
#pragma unroll
        for (int k = 0; k < 8; ++k) g[k] += dsj * c[k] / len;
      }
    }
    if (t == mp)
      for (int j = 0; j < n; ++j) {
        const float dsj = ds[j];
        const float* hs = a.h_spans + (int64_t(b) * n + j) * D;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int d = d0 + lane + 64 * k;
          if (d < D) g[k] = __builtin_fmaf(dsj, hs[d], g[k]);
        }
      }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int d = d0 + lane + 64 * k;
      if (d < D) out[d] = uint16_t(pack2<E>(g[k], 0.f) & 0xFFFFu);
    }
  }
}

}  // namespace

int launch_span(const kd_span_args& a, hipStream_t st) {
  hipLaunchKernelGGL(k_span_find, dim3(unsigned(a.B)), dim3(1024), size_t(2) * a.n_spans * sizeof(int), st, a);
  const dim3 pool(unsigned(a.n_spans + 1), unsigned(a.B), unsigned((a.D + 255) / 256));
  if (a.dtype == KD_BF16)
    hipLaunchKernelGGL(k_span_pool<BF16>, pool, dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL(k_span_pool<F16>, pool, dim3(512), 0, st, a);
  hipLaunchKernelGGL(k_span_score, dim3(unsigned(a.n_spans), unsigned(a.B)), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

int launch_span_bwd(const kd_span_args& a, hipStream_t st) {
  const dim3 grid(unsigned((a.T + 3) / 4), unsigned(a.B));
  if (a.dtype == KD_BF16) hipLaunchKernelGGL(k_span_bwd<BF16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(k_span_bwd<F16>, grid, dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
