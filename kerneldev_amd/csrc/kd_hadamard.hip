// Walsh-Hadamard incoherent processing of Q / K rows on gfx950.
//
// The reference names generate_hadamard_signs() / hadamard_transform()
// (README.md:68-71, :77) without code; the transform is defined here as
//   x R,  R = diag(s) H_d / sqrt(d),  H_d the Sylvester matrix, s in {+1,-1}^d
// and its inverse (used for gradients) g R^T = ((g H_d) / sqrt(d)) * s.
// Q R (K R)^T = Q K^T exactly in real arithmetic.
//
// Evaluation order is fixed so the result is bit-identical to the CPU
// restatement: signs (exact), butterflies h = 1, 2, ..., d/2 each rounded to
// fp32 ((a, b) -> (a + b, a - b)), one multiply by fp32(1/sqrt(d)), one
// rounding to the output dtype.  D/8 lanes hold one row, 8 elements each:
// strides 1, 2, 4 stay inside a lane, strides 8 .. d/2 pair lane t with
// lane t ^ (h / 8).  Optionally the kernel also records max |y| per (b, h)
// (the absmax the fp8 path scales by).
#include "kd_internal.h"

namespace kd {

constexpr int HAD_ITERS = 16;  // rows per thread (one chunk per block)

// One block transforms a contiguous chunk of ITERS * RPB rows, RPB per
// iteration, with the next iteration's row loaded while the current one is
// transformed.  The optional absmax is kept per thread as (b*H + h, max) over
// its rows, then reduced over the block, so a chunk inside one head costs one
// atomic (chunks that straddle heads flush per thread).
template <class E, int D, bool INV>
__global__ __launch_bounds__(256) void k_hadamard(kd_rot_args a) {
  constexpr int TPR = D / 8;         // lanes per row
  constexpr int RPB = 256 / TPR;     // rows per iteration
  constexpr int ITERS = HAD_ITERS;
  const int tid = threadIdx.x, seg = tid % TPR;
  const int64_t nrows = int64_t(a.B) * a.H * a.T;
  const int64_t row0 = int64_t(blockIdx.x) * (ITERS * RPB) + tid / TPR;

  float sg[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sg[j] = a.signs[seg * 8 + j];

  auto src = [&](int64_t row) {
    const int64_t r = row < nrows ? row : nrows - 1;  // idle lanes still join the shuffles
    const int t = int(r % a.T), bh = int(r / a.T), b = bh / a.H, h = bh % a.H;
    return static_cast<const uint16_t*>(a.x) + b * a.x_strides[0] + h * a.x_strides[1] + t * a.x_strides[2] +
           seg * 8;
  };
  int run_bh = -1;
  float run_m = 0.f;
  u32x4 xv = *reinterpret_cast<const u32x4*>(src(row0));
  for (int it = 0; it < ITERS; ++it) {
    const int64_t row = row0 + int64_t(it) * RPB;
    if (row - (tid / TPR) >= nrows) break;  // block-uniform: the chunk ran past the end
    u32x4 nxt = xv;
    if (it + 1 < ITERS) nxt = *reinterpret_cast<const u32x4*>(src(row + RPB));
    const bool valid = row < nrows;
    const int64_t r = valid ? row : nrows - 1;
    const int t = int(r % a.T), bh = int(r / a.T), b = bh / a.H, h = bh % a.H;
    float y[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      y[2 * w] = to_f32<E>(uint16_t(xv[w] & 0xFFFFu));
      y[2 * w + 1] = to_f32<E>(uint16_t(xv[w] >> 16));
    }
    if (!INV) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] *= sg[j];
    }
    // in-lane butterflies, strides 1, 2, 4
#pragma unroll
    for (int hs = 1; hs < 8; hs <<= 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j & hs) continue;
        const float u = y[j], v = y[j + hs];
        y[j] = u + v;
        y[j + hs] = u - v;
      }
    }
    // cross-lane butterflies, strides 8 .. D/2
#pragma unroll
    for (int m = 1; m < TPR; m <<= 1) {
      const bool upper = (seg & m) != 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float other = __shfl_xor(y[j], m, TPR);
        y[j] = upper ? other - y[j] : y[j] + other;
      }
    }
    // fp32(1 / sqrt(D)), correctly rounded
    constexpr float scale = D == 64 ? 0x1p-3f : 0x1.6a09e6p-4f;
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] *= scale;
    if (INV) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] *= sg[j];
    }
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) out[w] = pack2<E>(y[2 * w], y[2 * w + 1]);
    if (valid) {
      uint16_t* yp = static_cast<uint16_t*>(a.y) + b * a.y_strides[0] + h * a.y_strides[1] +
                     t * a.y_strides[2] + seg * 8;
      *reinterpret_cast<u32x4*>(yp) = out;
    }
    if (a.amax != nullptr && valid) {
      // |y| of the ROUNDED output (this lane's 8 elements)
      float m = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        m = fmaxf(m, fabsf(to_f32<E>(uint16_t(out[w] & 0xFFFFu))));
        m = fmaxf(m, fabsf(to_f32<E>(uint16_t(out[w] >> 16))));
      }
      if (bh != run_bh) {
        if (run_bh >= 0) atomicMax(reinterpret_cast<unsigned int*>(a.amax) + run_bh, __float_as_uint(run_m));
        run_bh = bh;
        run_m = 0.f;
      }
      run_m = fmaxf(run_m, m);
    }
    xv = nxt;
  }
  if (a.amax == nullptr) return;
  // block reduction when every thread's last head is the same (the usual case)
  __shared__ int s_bh[256];
  __shared__ float s_m[256];
  s_bh[tid] = run_bh;
  s_m[tid] = run_m;
  __syncthreads();
  const int bh0 = s_bh[0];
  bool same = true;
  for (int i = 0; i < 256; i += 64) same = same && __all(s_bh[i + (tid & 63)] == bh0);
  if (same) {
    if (bh0 < 0) return;
    if (tid < 64) {
      float m = fmaxf(fmaxf(s_m[tid], s_m[tid + 64]), fmaxf(s_m[tid + 128], s_m[tid + 192]));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      if (tid == 0) atomicMax(reinterpret_cast<unsigned int*>(a.amax) + bh0, __float_as_uint(m));
    }
  } else if (run_bh >= 0) {
    atomicMax(reinterpret_cast<unsigned int*>(a.amax) + run_bh, __float_as_uint(run_m));
  }
}

// ---- fp8 e4m3 quantisation per (b, h) -----------------------------------
// y = e4m3(clamp(fp32(x * inv), -448, 448)) with inv = fp32(448 / amax), round
// to nearest even (v_cvt_pk_fp8_f32 is OCP e4m3 on gfx950); scale = amax / 448.
template <class E, int D>
__global__ __launch_bounds__(256) void k_quant8(kd_quant_args a) {
  constexpr int TPR = D / 8;
  constexpr int RPB = 256 / TPR;
  const int tid = threadIdx.x, seg = tid % TPR;
  const int64_t row = int64_t(blockIdx.x) * RPB + tid / TPR;
  const int64_t nrows = int64_t(a.B) * a.H * a.T;
  if (row >= nrows) return;
  const int t = int(row % a.T);
  const int bh = int(row / a.T);
  const int b = bh / a.H, h = bh % a.H;
  const float am = a.amax[bh];
  const float safe = am > 0.f ? am : 448.f;
  const float inv = 448.f / safe;  // IEEE division (no fast-math)
  if (t == 0 && seg == 0) a.scale[bh] = safe / 448.f;
  const uint16_t* xp = static_cast<const uint16_t*>(a.x) + b * a.x_strides[0] + h * a.x_strides[1] +
                       t * a.x_strides[2] + seg * 8;
  const u32x4 xv = *reinterpret_cast<const u32x4*>(xp);
  uint32_t w[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float f[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f[2 * j] = to_f32<E>(uint16_t(xv[2 * k + j] & 0xFFFFu)) * inv;
      f[2 * j + 1] = to_f32<E>(uint16_t(xv[2 * k + j] >> 16)) * inv;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = fminf(fmaxf(f[j], -448.f), 448.f);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
    w[k] = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], lo, true));
  }
  uint8_t* yp = a.y + row * D + seg * 8;
  *reinterpret_cast<u32x2*>(yp) = u32x2{w[0], w[1]};
}

template <class E, int D>
static void launch_quant_t(const kd_quant_args& a, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  hipLaunchKernelGGL((k_quant8<E, D>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
}

int launch_quant(const kd_quant_args& a, hipStream_t st) {
  if (a.dtype == KD_BF16) {
    if (a.D == 64) launch_quant_t<BF16, 64>(a, st);
    else launch_quant_t<BF16, 128>(a, st);
  } else {
    if (a.D == 64) launch_quant_t<F16, 64>(a, st);
    else launch_quant_t<F16, 128>(a, st);
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

template <class E, int D, bool INV>
static void launch_rot_t(const kd_rot_args& a, hipStream_t st) {
  constexpr int CHUNK = HAD_ITERS * (256 / (D / 8));
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  hipLaunchKernelGGL((k_hadamard<E, D, INV>), dim3(unsigned((rows + CHUNK - 1) / CHUNK)), dim3(256), 0, st, a);
}

int launch_hadamard(const kd_rot_args& a, hipStream_t st) {
#define KD_ROT(E_, D_)                                          \
  if (a.inverse) launch_rot_t<E_, D_, true>(a, st);             \
  else launch_rot_t<E_, D_, false>(a, st);
  if (a.dtype == KD_BF16) {
    if (a.D == 64) { KD_ROT(BF16, 64) } else { KD_ROT(BF16, 128) }
  } else {
    if (a.D == 64) { KD_ROT(F16, 64) } else { KD_ROT(F16, 128) }
  }
#undef KD_ROT
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
