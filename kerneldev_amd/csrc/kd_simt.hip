// Attention in fp32 arithmetic on the vector ALUs, for the case the MFMA
// kernels are not built for: fp32 inputs at head dim 16 through the C ABI
// (the reference's precision="ieee" / "tf32" dots, original_kernel.py:452,
// :569, :1239, :1331-1333, :1425, :1517-1523, here in full fp32; kd_f32w.hip
// takes fp32 at 32, 64, 128, 256), plus Delta for fp32 inputs at every head dim.  Same
// algebra, plan and masks as the MFMA kernels:
//   forward   O = softmax2(S c) V, LSE2 = m + log2 l      (:279-626)
//   Delta     rowsum(O * dO)                              (:649-710)
//   dQ        P = exp2(S c - LSE), dS = P (dP - Delta), dQ = sm_scale dS K  (:1173-1336)
//   dK / dV   dV = P^T dO, dK = sm_scale dS^T Q            (:1339-1525)
// c = sm_scale log2(e) in fp32.  Only non-empty 64 x 64 tiles are visited;
// PARTIAL tiles evaluate the mask rule allow() per score from the plan's token
// codes, FULL tiles skip it.
//
// Layout: one workgroup per (64-row tile, b, h).  G = max(1, D / 32) lanes
// share one row, each owning DL = D / G (16 or 32) consecutive columns in registers;
// dot products end with a G-lane xor reduction.  The streamed operand tiles
// go through LDS in fp32, 32 rows at a time (2 x 32 x D floats, 64 KiB at
// D = 256).  Every key of a sub-tile is read by all rows of the workgroup
// (an LDS broadcast), so LDS traffic per FMA is one float.
#include "kd_internal.h"

namespace kd {

template <class E> struct Elem;
template <> struct Elem<F32> { typedef float T; };

template <class E> KD_DEV float ld(const void* p, int64_t i);
template <> KD_DEV float ld<F32>(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }

// store x at element i of p (the residual arguments are for 16-bit element types)
template <class E> KD_DEV void st(void* p, int64_t i, float x, void* lo = nullptr, int64_t li = 0);
template <> KD_DEV void st<F32>(void* p, int64_t i, float x, void*, int64_t) { static_cast<float*>(p)[i] = x; }

template <int G> KD_DEV float group_sum(float x) {
#pragma unroll
  for (int o = 1; o < G; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

template <int D> struct Shape {
  static constexpr int G = D >= 32 ? D / 32 : 1;  // lanes per row
  static constexpr int DL = D / G;                // columns per lane
  static constexpr int NT = 64 * G;               // threads per workgroup
  static constexpr int SUB = 32;                  // streamed rows per LDS sub-tile
};

// Copies rows r0 .. r0 + SUB - 1 of a [T, D] slice (row stride rs elements)
// into s[SUB][D] as fp32; rows at or beyond T become zero.
template <class E, int D>
KD_DEV void fill(float (*s)[D], const void* base, int64_t rs, int r0, int T, int tid) {
  using S = Shape<D>;
  for (int e = tid; e < S::SUB * D; e += S::NT) {
    const int r = e / D, c = e % D, t = r0 + r;
    s[r][c] = t < T ? ld<E>(base, int64_t(t) * rs + c) : 0.f;
  }
}
KD_DEV void fill_vec(float* s, const float* base, int r0, int T, int tid, int nt, float dflt) {
  for (int r = tid; r < Shape<64>::SUB; r += nt) s[r] = r0 + r < T ? base[r0 + r] : dflt;
}

// token codes of rows r0 .. r0 + SUB - 1 (0 past T: allow nothing)
KD_DEV void fill_codes(uint32_t* s, const uint32_t* base, int r0, int T, int tid, int nt) {
  for (int r = tid; r < Shape<64>::SUB; r += nt) s[r] = r0 + r < T ? base[r0 + r] : 0u;
}

// ------------------------------------------------------------------ forward
template <class E, int D>
__global__ __launch_bounds__(Shape<D>::NT) void k_fwd_simt(AttnArgs a, const uint8_t* __restrict__ cls,
                                                           const uint32_t* __restrict__ codes, int nT) {
  using S = Shape<D>;
  constexpr int G = S::G, DL = S::DL, SUB = S::SUB;
  __shared__ float sk[SUB][D], sv[SUB][D];
  __shared__ uint32_t skc[SUB];
  const int qt = blockIdx.x, b = blockIdx.y, h = blockIdx.z, bh = b * a.H + h;
  const int tid = threadIdx.x, row = tid / G, g = tid % G, i = qt * 64 + row, T = a.T;
  const bool valid = i < T;
  const float c = a.sm_scale * 1.4426950408889634f;
  const void* qb = static_cast<const char*>(a.q) + (b * a.q_strides[0] + h * a.q_strides[1]) * int64_t(sizeof(typename Elem<E>::T));
  const void* kb = static_cast<const char*>(a.k) + (b * a.k_strides[0] + h * a.k_strides[1]) * int64_t(sizeof(typename Elem<E>::T));
  const void* vb = static_cast<const char*>(a.v) + (b * a.v_strides[0] + h * a.v_strides[1]) * int64_t(sizeof(typename Elem<E>::T));
  float q[DL], o[DL];
#pragma unroll
  for (int d = 0; d < DL; ++d) {
    q[d] = valid ? ld<E>(qb, int64_t(i) * a.q_strides[2] + g * DL + d) * c : 0.f;  // scores in log2 units
    o[d] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  const uint32_t* codes_b = codes + int64_t(b) * T;
  const uint32_t qc = valid ? codes_b[i] : 0u;
  const int64_t trow = int64_t(b) * nT + qt;
  for (int kt = 0; kt < nT; ++kt) {
    const uint8_t cl = cls[trow * nT + kt];
    if (cl == TILE_EMPTY) continue;  // uniform
    const bool partial = cl == TILE_PARTIAL;
    for (int half = 0; half < 2; ++half) {
      const int j0 = kt * 64 + half * SUB;
      __syncthreads();
      fill<E, D>(sk, kb, a.k_strides[2], j0, T, tid);
      fill<E, D>(sv, vb, a.v_strides[2], j0, T, tid);
      fill_codes(skc, codes_b, j0, T, tid, S::NT);
      __syncthreads();
      float s[SUB];  // fully unrolled loops keep s in registers
      float mx = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < SUB; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < DL; ++d) acc = __builtin_fmaf(q[d], sk[j][g * DL + d], acc);
        acc = group_sum<G>(acc);
        s[j] = (!partial || allow(qc, skc[j], i, j0 + j)) ? acc : -__builtin_inff();
        mx = fmaxf(mx, s[j]);
      }
      const float m_new = fmaxf(m, mx);
      if (m_new == -__builtin_inff()) continue;  // nothing allowed so far in this row
      const float alpha = fast_exp2(m - m_new);  // 0 when m == -inf
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DL; ++d) o[d] *= alpha;
      m = m_new;
#pragma unroll
      for (int j = 0; j < SUB; ++j) {
        const float p = fast_exp2(s[j] - m);  // 0 for masked keys
        l += p;
#pragma unroll
        for (int d = 0; d < DL; ++d) o[d] = __builtin_fmaf(p, sv[j][g * DL + d], o[d]);
      }
    }
  }
  if (!valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int64_t ob = b * a.o_strides[0] + h * a.o_strides[1] + int64_t(i) * a.o_strides[2] + g * DL;
  const int64_t lb = (int64_t(bh) * T + i) * D + g * DL;  // o_lo is contiguous [B, H, T, D]
#pragma unroll
  for (int d = 0; d < DL; ++d) st<E>(a.o, ob + d, o[d] * inv, a.o_lo, lb + d);
  if (g == 0 && a.lse != nullptr) a.lse[int64_t(bh) * T + i] = l > 0.f ? m + fast_log2(l) : -__builtin_inff();
}

// -------------------------------------------------------------------- Delta
// workspace: -Delta, then -LSE / c (the forms the MFMA dK/dV kernel reads);
// the fp32 kernels read -Delta and the LSE itself.  DeltaShape<D>::G lanes share
// a row, each reading EL consecutive elements (coalesced), and the row's sum
// ends in a G-lane xor reduction.
template <int D> struct DeltaShape {
  static constexpr int G = D >= 64 ? 16 : D / 4;  // lanes per row
  static constexpr int EL = D / G;                // elements per lane (4 .. 16)
  static constexpr int RPB = 256 / G;             // rows per 256-thread block
};
template <class E, int D>
__global__ __launch_bounds__(256) void k_delta_simt(AttnArgs a) {
  using S = DeltaShape<D>;
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  const int64_t r = int64_t(blockIdx.x) * S::RPB + threadIdx.x / S::G;
  const int g = threadIdx.x % S::G;
  const bool valid = r < rows;  // (every lane takes part in the reduction below)
  float sum = 0.f;
  if (valid) {
    const int t = int(r % a.T), bh = int(r / a.T), b = bh / a.H, h = bh % a.H;
    const int64_t ob = b * a.o_strides[0] + h * a.o_strides[1] + int64_t(t) * a.o_strides[2] + g * S::EL;
    const int64_t db = b * a.do_strides[0] + h * a.do_strides[1] + int64_t(t) * a.do_strides[2] + g * S::EL;
#pragma unroll
    for (int d = 0; d < S::EL; ++d) {
      float o = ld<E>(a.o, ob + d);
      if (a.o_lo != nullptr) o += ld<E>(a.o_lo, r * D + g * S::EL + d);  // 16-bit O only (the C ABI refuses it for fp32)
      sum = __builtin_fmaf(o, ld<E>(a.dout, db + d), sum);
    }
  }
  sum = group_sum<S::G>(sum);
  if (!valid || g != 0) return;
  const float c = a.sm_scale * 1.4426950408889634f;
  const float l = a.lse[r];
  a.delta[r] = -sum;
  a.delta[rows + r] = l == -__builtin_inff() ? -__builtin_inff() : -l / c;
}

// ----------------------------------------------------------------------- dQ
template <class E, int D>
__global__ __launch_bounds__(Shape<D>::NT) void k_dq_simt(AttnArgs a, const uint8_t* __restrict__ cls,
                                                          const uint32_t* __restrict__ codes, int nT) {
  using S = Shape<D>;
  constexpr int G = S::G, DL = S::DL, SUB = S::SUB;
  __shared__ float sk[SUB][D], sv[SUB][D];
  __shared__ uint32_t skc[SUB];
  const int qt = blockIdx.x, b = blockIdx.y, h = blockIdx.z, bh = b * a.H + h;
  const int tid = threadIdx.x, row = tid / G, g = tid % G, i = qt * 64 + row, T = a.T;
  const bool valid = i < T;
  const float c = a.sm_scale * 1.4426950408889634f;
  constexpr int64_t ES = sizeof(typename Elem<E>::T);
  const void* qb = static_cast<const char*>(a.q) + (b * a.q_strides[0] + h * a.q_strides[1]) * ES;
  const void* kb = static_cast<const char*>(a.k) + (b * a.k_strides[0] + h * a.k_strides[1]) * ES;
  const void* vb = static_cast<const char*>(a.v) + (b * a.v_strides[0] + h * a.v_strides[1]) * ES;
  const void* dob = static_cast<const char*>(a.dout) + (b * a.do_strides[0] + h * a.do_strides[1]) * ES;
  float q[DL], dov[DL], dq[DL];
#pragma unroll
  for (int d = 0; d < DL; ++d) {
    q[d] = valid ? ld<E>(qb, int64_t(i) * a.q_strides[2] + g * DL + d) * c : 0.f;
    dov[d] = valid ? ld<E>(dob, int64_t(i) * a.do_strides[2] + g * DL + d) : 0.f;
    dq[d] = 0.f;
  }
  const float l = valid ? a.lse[int64_t(bh) * T + i] : -__builtin_inff();
  const float lse = l == -__builtin_inff() ? __builtin_inff() : l;  // fully masked rows: P = 0
  const float delta = valid ? -a.delta[int64_t(bh) * T + i] : 0.f;
  const uint32_t* codes_b = codes + int64_t(b) * T;
  const uint32_t qc = valid ? codes_b[i] : 0u;
  const int64_t trow = int64_t(b) * nT + qt;
  for (int kt = 0; kt < nT; ++kt) {
    const uint8_t cl = cls[trow * nT + kt];
    if (cl == TILE_EMPTY) continue;
    const bool partial = cl == TILE_PARTIAL;
    for (int half = 0; half < 2; ++half) {
      const int j0 = kt * 64 + half * SUB;
      __syncthreads();
      fill<E, D>(sk, kb, a.k_strides[2], j0, T, tid);
      fill<E, D>(sv, vb, a.v_strides[2], j0, T, tid);
      fill_codes(skc, codes_b, j0, T, tid, S::NT);
      __syncthreads();
#pragma unroll 2
      for (int j = 0; j < SUB; ++j) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < DL; ++d) {
          s = __builtin_fmaf(q[d], sk[j][g * DL + d], s);
          dp = __builtin_fmaf(dov[d], sv[j][g * DL + d], dp);
        }
        s = group_sum<G>(s);
        dp = group_sum<G>(dp);
        const float p = (!partial || allow(qc, skc[j], i, j0 + j)) ? fast_exp2(s - lse) : 0.f;
        const float ds = p * (dp - delta);
#pragma unroll
        for (int d = 0; d < DL; ++d) dq[d] = __builtin_fmaf(ds, sk[j][g * DL + d], dq[d]);
      }
    }
  }
  if (!valid) return;
  const int64_t ob = b * a.dq_strides[0] + h * a.dq_strides[1] + int64_t(i) * a.dq_strides[2] + g * DL;
#pragma unroll
  for (int d = 0; d < DL; ++d) st<E>(a.dq, ob + d, dq[d] * a.sm_scale);
}

// -------------------------------------------------------------------- dK/dV
template <class E, int D>
__global__ __launch_bounds__(Shape<D>::NT) void k_dkdv_simt(AttnArgs a, const uint8_t* __restrict__ cls,
                                                            const uint32_t* __restrict__ codes, int nT) {
  using S = Shape<D>;
  constexpr int G = S::G, DL = S::DL, SUB = S::SUB;
  __shared__ float sq[SUB][D], sdo[SUB][D];
  __shared__ float slse[SUB], sdl[SUB];
  __shared__ uint32_t sqc[SUB];
  const int kt = blockIdx.x, b = blockIdx.y, h = blockIdx.z, bh = b * a.H + h;
  const int tid = threadIdx.x, row = tid / G, g = tid % G, j = kt * 64 + row, T = a.T;
  const bool valid = j < T;
  const float c = a.sm_scale * 1.4426950408889634f;
  constexpr int64_t ES = sizeof(typename Elem<E>::T);
  const void* qb = static_cast<const char*>(a.q) + (b * a.q_strides[0] + h * a.q_strides[1]) * ES;
  const void* kb = static_cast<const char*>(a.k) + (b * a.k_strides[0] + h * a.k_strides[1]) * ES;
  const void* vb = static_cast<const char*>(a.v) + (b * a.v_strides[0] + h * a.v_strides[1]) * ES;
  const void* dob = static_cast<const char*>(a.dout) + (b * a.do_strides[0] + h * a.do_strides[1]) * ES;
  float k[DL], v[DL], dk[DL], dv[DL];
#pragma unroll
  for (int d = 0; d < DL; ++d) {
    k[d] = valid ? ld<E>(kb, int64_t(j) * a.k_strides[2] + g * DL + d) * c : 0.f;
    v[d] = valid ? ld<E>(vb, int64_t(j) * a.v_strides[2] + g * DL + d) : 0.f;
    dk[d] = dv[d] = 0.f;
  }
  const float* lse_g = a.lse + int64_t(bh) * T;
  const float* dl_g = a.delta + int64_t(bh) * T;  // -Delta
  const uint32_t* codes_b = codes + int64_t(b) * T;
  const uint32_t kc = valid ? codes_b[j] : 0u;
  for (int qt = 0; qt < nT; ++qt) {
    const int64_t trow = int64_t(b) * nT + qt;
    const uint8_t cl = cls[trow * nT + kt];
    if (cl == TILE_EMPTY) continue;
    const bool partial = cl == TILE_PARTIAL;
    for (int half = 0; half < 2; ++half) {
      const int i0 = qt * 64 + half * SUB;
      __syncthreads();
      fill<E, D>(sq, qb, a.q_strides[2], i0, T, tid);
      fill<E, D>(sdo, dob, a.do_strides[2], i0, T, tid);
      fill_vec(slse, lse_g, i0, T, tid, S::NT, -__builtin_inff());
      fill_vec(sdl, dl_g, i0, T, tid, S::NT, 0.f);
      fill_codes(sqc, codes_b, i0, T, tid, S::NT);
      __syncthreads();
#pragma unroll 2
      for (int r = 0; r < SUB; ++r) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < DL; ++d) {
          s = __builtin_fmaf(k[d], sq[r][g * DL + d], s);
          dp = __builtin_fmaf(v[d], sdo[r][g * DL + d], dp);
        }
        s = group_sum<G>(s);
        dp = group_sum<G>(dp);
        const float l = slse[r];
        const bool ok = !partial || allow(sqc[r], kc, i0 + r, j);
        const float p = (ok && l != -__builtin_inff()) ? fast_exp2(s - l) : 0.f;
        const float ds = p * (dp + sdl[r]);  // sdl holds -Delta
#pragma unroll
        for (int d = 0; d < DL; ++d) {
          dv[d] = __builtin_fmaf(p, sdo[r][g * DL + d], dv[d]);
          dk[d] = __builtin_fmaf(ds, sq[r][g * DL + d], dk[d]);
        }
      }
    }
  }
  if (!valid) return;
  const int64_t kb_o = b * a.dk_strides[0] + h * a.dk_strides[1] + int64_t(j) * a.dk_strides[2] + g * DL;
  const int64_t vb_o = b * a.dv_strides[0] + h * a.dv_strides[1] + int64_t(j) * a.dv_strides[2] + g * DL;
#pragma unroll
  for (int d = 0; d < DL; ++d) {
    st<E>(a.dk, kb_o + d, dk[d] * a.sm_scale);
    st<E>(a.dv, vb_o + d, dv[d]);
  }
}

// ---------------------------------------------------------------- launchers
template <class E, int D>
static void launch_simt(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const dim3 grid(unsigned(L.nT), unsigned(a.B), unsigned(a.H));
  const uint8_t* cls = plan + L.cls;
  const uint32_t* codes = reinterpret_cast<const uint32_t*>(plan + L.codes);
  if (which == 0) hipLaunchKernelGGL((k_fwd_simt<E, D>), grid, dim3(Shape<D>::NT), 0, st, a, cls, codes, L.nT);
  if (which == 1) {
    const int64_t rows = int64_t(a.B) * a.H * a.T;
    constexpr int rpb = DeltaShape<D>::RPB;
    hipLaunchKernelGGL((k_delta_simt<E, D>), dim3(unsigned((rows + rpb - 1) / rpb)), dim3(256), 0, st, a);
  }
  if (which == 2) hipLaunchKernelGGL((k_dq_simt<E, D>), grid, dim3(Shape<D>::NT), 0, st, a, cls, codes, L.nT);
  if (which == 3) hipLaunchKernelGGL((k_dkdv_simt<E, D>), grid, dim3(Shape<D>::NT), 0, st, a, cls, codes, L.nT);
}

template <class E>
static void launch_simt_d(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  switch (a.D) {
    case 16: launch_simt<E, 16>(which, a, plan, st); break;
    case 32: launch_simt<E, 32>(which, a, plan, st); break;
    case 64: launch_simt<E, 64>(which, a, plan, st); break;
    case 128: launch_simt<E, 128>(which, a, plan, st); break;
    default: launch_simt<E, 256>(which, a, plan, st); break;
  }
}

// fp32 inputs (16-bit inputs run on the MFMA kernels at every head dim)
bool use_simt(const AttnArgs& a) { return a.dtype == KD_F32; }

// which: 0 forward, 1 Delta, 2 dQ, 3 dK/dV
int launch_simt_kernel(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (which != 1 && use_f32mma(a)) return launch_f32mma(which, a, plan, st);
  launch_simt_d<F32>(which, a, plan, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
