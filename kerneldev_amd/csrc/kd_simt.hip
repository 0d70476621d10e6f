// fp32 inputs: Delta on the vector ALUs (the reference's _flash_attn_bwd_precompute,
// original_kernel.py:649-710, in fp32) and the dispatch of the fp32 attention
// kernels, which run on the fp32 MFMA at every head dim (kd_f32w.hip).
//   Delta     rowsum(O * dO), written as -Delta, then -LSE / c (c = sm_scale log2(e))
#include "kd_internal.h"

namespace kd {

template <int G> KD_DEV float group_sum(float x) {
#pragma unroll
  for (int o = 1; o < G; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
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
    // 16-byte reads: rows and the lane's EL (a multiple of 4) elements are
    // 16-byte aligned (the C ABI's stride and base checks); fp32 inputs carry
    // no O residual (the C ABI refuses o_lo for them)
    const float* op = static_cast<const float*>(a.o) + ob;
    const float* dp = static_cast<const float*>(a.dout) + db;
#pragma unroll
    for (int d = 0; d < S::EL; d += 4) {
      const f32x4 o = *reinterpret_cast<const f32x4*>(op + d);
      const f32x4 x = *reinterpret_cast<const f32x4*>(dp + d);
#pragma unroll
      for (int j = 0; j < 4; ++j) sum = __builtin_fmaf(o[j], x[j], sum);
    }
  }
  sum = group_sum<S::G>(sum);
  if (!valid || g != 0) return;
  const float c = a.sm_scale * 1.4426950408889634f;
  const float l = a.lse[r];
  a.delta[r] = -sum;
  a.delta[rows + r] = l == -__builtin_inff() ? -__builtin_inff() : -l / c;
}

// ---------------------------------------------------------------- launchers
template <int D>
static void launch_delta_f32(const AttnArgs& a, hipStream_t st) {
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  constexpr int rpb = DeltaShape<D>::RPB;
  hipLaunchKernelGGL((k_delta_simt<F32, D>), dim3(unsigned((rows + rpb - 1) / rpb)), dim3(256), 0, st, a);
}

// fp32 inputs (16-bit inputs run on the 16-bit MFMA kernels)
bool use_simt(const AttnArgs& a) { return a.dtype == KD_F32; }

// which: 0 forward, 1 Delta, 2 dQ, 3 dK/dV
int launch_simt_kernel(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (which != 1) return launch_f32mma(which, a, plan, st);
  switch (a.D) {
    case 16: launch_delta_f32<16>(a, st); break;
    case 32: launch_delta_f32<32>(a, st); break;
    case 64: launch_delta_f32<64>(a, st); break;
    case 128: launch_delta_f32<128>(a, st); break;
    default: launch_delta_f32<256>(a, st); break;
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
