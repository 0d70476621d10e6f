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
// rounding to the output dtype (none for fp32).  D/8 lanes hold one row
// (D = 16 .. 256), 8 elements each: strides 1, 2, 4 stay inside a lane,
// strides 8 .. d/2 pair lane t with lane t ^ (h / 8).  Optionally the kernel also records max |y| per (b, h)
// (the absmax the fp8 path scales by).
#include <type_traits>

#include "kd_internal.h"

namespace kd {


// Lane exchanges inside a row's D/8 lanes through DPP (no LDS traffic):
// partner lane l ^ m for m = 1, 2 (quad_perm), 4 (half-row mirror, then
// quad reverse) and 8 (row mirror, then half-row mirror); 16 (D = 256, rows
// of 32 lanes) crosses DPP rows and goes through ds_bpermute.
template <int M>
KD_DEV float xor_lane(float v) {
  const int x = __float_as_int(v);
  if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  if constexpr (M == 4) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);  // row_half_mirror
    return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, false));  // quad_perm [3,2,1,0]
  }
  if constexpr (M == 8) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);  // row_mirror
    return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, false));
  }
  return __shfl_xor(v, M, 64);
}

// Eight consecutive elements of a row: one 16-byte word for 16-bit types, two for fp32.
template <class E> struct Row8 { u32x4 w[1]; };
template <> struct Row8<F32> { u32x4 w[2]; };
template <class E> KD_DEV Row8<E> load_row8(const void* base, int64_t off) {  // off in elements
  Row8<E> r;
  constexpr int NW = sizeof(Row8<E>) / 16;
  const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + off * (NW == 1 ? 2 : 4));
#pragma unroll
  for (int k = 0; k < NW; ++k) r.w[k] = p[k];
  return r;
}
template <class E> KD_DEV void unpack_row8(const Row8<E>& r, float (&y)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    y[2 * w] = to_f32<E>(uint16_t(r.w[0][w] & 0xFFFFu));
    y[2 * w + 1] = to_f32<E>(uint16_t(r.w[0][w] >> 16));
  }
}
template <> KD_DEV void unpack_row8<F32>(const Row8<F32>& r, float (&y)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = __uint_as_float(r.w[j >> 2][j & 3]);
}
// round y to E, store it, and max |stored value| into m
template <class E> KD_DEV void store_row8(void* base, int64_t off, const float (&y)[8], float& m) {
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) out[w] = pack2<E>(y[2 * w], y[2 * w + 1]);
  *reinterpret_cast<u32x4*>(static_cast<char*>(base) + off * 2) = out;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    m = fmaxf(m, fmaxf(fabsf(to_f32<E>(uint16_t(out[w] & 0xFFFFu))), fabsf(to_f32<E>(uint16_t(out[w] >> 16)))));
}
template <> KD_DEV void store_row8<F32>(void* base, int64_t off, const float (&y)[8], float& m) {
  u32x4* p = reinterpret_cast<u32x4*>(static_cast<char*>(base) + off * 4);
  p[0] = u32x4{__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3])};
  p[1] = u32x4{__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]), __float_as_uint(y[7])};
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(y[j]));
}

// fp32(1 / sqrt(D)), correctly rounded
template <int D> constexpr float inv_sqrt_d() {
  return D == 16 ? 0x1p-2f : D == 32 ? 0x1.6a09e6p-3f : D == 64 ? 0x1p-3f : D == 128 ? 0x1.6a09e6p-4f : 0x1p-4f;
}

// One block = ITERS x RPB consecutive rows of one (b, h) (grid: row chunks x
// B*H), so the row index needs no division and the optional absmax is one
// block reduction and one atomic per block.  Without the absmax a block does
// two RPB-row steps (measured 5% faster than one); with it, 16 steps, so that
// each (b, h) collects few atomics.
template <class E, int D, bool INV, int ITERS>
__global__ __launch_bounds__(256) void k_hadamard(kd_rot_args a) {
  constexpr int TPR = D / 8;         // lanes per row
  constexpr int RPB = 256 / TPR;     // rows per step
  const int tid = threadIdx.x, seg = tid % TPR;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int64_t xb = b * a.x_strides[0] + h * a.x_strides[1] + seg * 8;  // element offsets
  const int64_t yb = b * a.y_strides[0] + h * a.y_strides[1] + seg * 8;
  float sg[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sg[j] = a.signs[seg * 8 + j];
  float m = 0.f;  // max |y| of the rounded outputs of this lane's rows
  const int t0 = blockIdx.x * (ITERS * RPB) + tid / TPR;
  Row8<E> xv = load_row8<E>(a.x, xb + int64_t(t0 < a.T ? t0 : a.T - 1) * a.x_strides[2]);
#pragma unroll 1
  for (int it = 0; it < ITERS; ++it) {
    const int t = t0 + it * RPB;
    if (t - tid / TPR >= a.T) break;  // block-uniform: the chunk ran past the end
    const bool valid = t < a.T;       // idle lanes still join the exchanges
    Row8<E> nxt = xv;
    if (it + 1 < ITERS) {
      const int tn = t + RPB;
      nxt = load_row8<E>(a.x, xb + int64_t(tn < a.T ? tn : a.T - 1) * a.x_strides[2]);
    }
    float y[8];
    unpack_row8<E>(xv, y);
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
    // cross-lane butterflies, strides 8 .. D/2: the lower lane of a pair keeps
    // y + partner, the upper one partner - y; fma(y, +-1, partner) is exactly that sum
    auto cross = [&](auto m_tag) {
      constexpr int M = decltype(m_tag)::value;
      const float sgn = (seg & M) ? -1.f : 1.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = __builtin_fmaf(y[j], sgn, xor_lane<M>(y[j]));
    };
    if constexpr (TPR > 1) cross(std::integral_constant<int, 1>{});
    if constexpr (TPR > 2) cross(std::integral_constant<int, 2>{});
    if constexpr (TPR > 4) cross(std::integral_constant<int, 4>{});
    if constexpr (TPR > 8) cross(std::integral_constant<int, 8>{});
    if constexpr (TPR > 16) cross(std::integral_constant<int, 16>{});
    constexpr float scale = inv_sqrt_d<D>();
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] *= scale;
    if (INV) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] *= sg[j];
    }
    if (valid) {
      float mm = 0.f;
      store_row8<E>(a.y, yb + int64_t(t) * a.y_strides[2], y, mm);
      if (a.amax != nullptr) m = fmaxf(m, mm);
    }
    xv = nxt;
  }
  if (a.amax == nullptr) return;  // uniform
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __shared__ float s_m[4];
  if ((tid & 63) == 0) s_m[tid >> 6] = m;
  __syncthreads();
  if (tid == 0)
    atomicMax(reinterpret_cast<unsigned int*>(a.amax) + bh,
              __float_as_uint(fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]))));
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

// ---- per-(b, h) max |x| -----------------------------------------------------
// S B H workgroups, S a (b, h): the S 1024-thread workgroups stride over its
// T x D slice in 16-byte chunks (8 elements), four chunks in flight per
// thread; S is chosen so that about 256 workgroups (one a CU, 16 waves each)
// fill the chip whatever B H is, with few atomics meeting at one address.  The magnitudes of non-negative bf16 / fp16 values order as their
// bit patterns do, so the reduction runs on 15-bit integers (the sign bit
// cleared); a workgroup converts its maximum to fp32 once and folds it into
// amax[b H + h] with an integer atomic max on the float's bits, which
// non-negative floats order by too: exact, and independent of the order of
// the fold.  k_zero_f32 clears amax first, on the same stream.  A workgroup
// first reads amax[b H + h] and skips the atomic when the value there is
// already at least its own: amax only grows, so a stale read can only cost an
// atomic, never lose one.  (Device-scope atomics from the eight XCDs onto the
// few cache lines of amax serialise: 16 times the workgroups, four thousand
// atomics onto 64 heads, took several times as long as the reads.)
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ p, int n) {
  const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
  if (i < n) p[i] = 0.f;
}

template <class E>
__global__ __launch_bounds__(1024) void k_absmax(kd_quant_args a, float* __restrict__ amax, int cpr_log2, int S) {
  const int bh = int(blockIdx.x) / S, part = int(blockIdx.x) % S, b = bh / a.H, h = bh % a.H, tid = threadIdx.x;
  const int64_t n = int64_t(a.T) << cpr_log2;  // chunks in the slice (D / 8 a row, a power of two)
  const int cmask = (1 << cpr_log2) - 1;
  const uint16_t* base = static_cast<const uint16_t*>(a.x) + b * a.x_strides[0] + h * a.x_strides[1];
  uint32_t m = 0;
  auto fold = [&](const u32x4& v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) m = max(m, max(v[j] & 0x7FFFu, (v[j] >> 16) & 0x7FFFu));
  };
  auto chunk = [&](int64_t i) {
    return *reinterpret_cast<const u32x4*>(base + (i >> cpr_log2) * a.x_strides[2] + (int(i) & cmask) * 8);
  };
  const int64_t step = int64_t(S) * 1024;
  int64_t i = int64_t(part) * 1024 + tid;
  for (; i + 3 * step < n; i += 4 * step) {
    const u32x4 v0 = chunk(i), v1 = chunk(i + step), v2 = chunk(i + 2 * step), v3 = chunk(i + 3 * step);
    fold(v0);
    fold(v1);
    fold(v2);
    fold(v3);
  }
  for (; i < n; i += step) fold(chunk(i));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, uint32_t(__shfl_xor(int(m), off, 64)));
  __shared__ uint32_t s_m[16];
  if ((tid & 63) == 0) s_m[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) r = max(r, s_m[w]);
    unsigned int* dst = reinterpret_cast<unsigned int*>(amax) + bh;
    const unsigned int bits = __float_as_uint(to_f32<E>(uint16_t(r)));
    if (r != 0u && __hip_atomic_load(dst, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < bits) atomicMax(dst, bits);
  }
}

int launch_absmax(const kd_quant_args& a, float* amax, hipStream_t st) {
  const int bh = a.B * a.H;
  const int cpr_log2 = __builtin_ctz(unsigned(a.D / 8));
  const int64_t chunks = int64_t(a.T) << cpr_log2;
  const int64_t per_bh = (chunks + 4095) / 4096;  // workgroups that each take four chunks a thread
  const int want = bh >= 256 ? 1 : 256 / bh;
  const int S = int(per_bh < want ? per_bh : want);
  hipLaunchKernelGGL(k_zero_f32, dim3(unsigned((bh + 255) / 256)), dim3(256), 0, st, amax, bh);
  const dim3 grid(unsigned(int64_t(S) * bh)), block(1024);
  if (a.dtype == KD_BF16) hipLaunchKernelGGL(k_absmax<BF16>, grid, block, 0, st, a, amax, cpr_log2, S);
  else hipLaunchKernelGGL(k_absmax<F16>, grid, block, 0, st, a, amax, cpr_log2, S);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
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
    else if (a.D == 128) launch_quant_t<BF16, 128>(a, st);
    else launch_quant_t<BF16, 256>(a, st);
  } else {
    if (a.D == 64) launch_quant_t<F16, 64>(a, st);
    else if (a.D == 128) launch_quant_t<F16, 128>(a, st);
    else launch_quant_t<F16, 256>(a, st);
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

template <class E, int D, bool INV>
static void launch_rot_t(const kd_rot_args& a, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const dim3 block(256);
  if (a.amax == nullptr) {
    // two row steps per block, the second row's load issued before the first's butterflies
    hipLaunchKernelGGL((k_hadamard<E, D, INV, 2>), dim3(unsigned((a.T + 2 * RPB - 1) / (2 * RPB)), unsigned(a.B * a.H)),
                       block, 0, st, a);
  } else {
    constexpr int CH = 16 * RPB;
    hipLaunchKernelGGL((k_hadamard<E, D, INV, 16>), dim3(unsigned((a.T + CH - 1) / CH), unsigned(a.B * a.H)), block,
                       0, st, a);
  }
}

template <class E, bool INV>
static void launch_rot_d(const kd_rot_args& a, hipStream_t st) {
  switch (a.D) {
    case 16: launch_rot_t<E, 16, INV>(a, st); break;
    case 32: launch_rot_t<E, 32, INV>(a, st); break;
    case 64: launch_rot_t<E, 64, INV>(a, st); break;
    case 128: launch_rot_t<E, 128, INV>(a, st); break;
    default: launch_rot_t<E, 256, INV>(a, st); break;
  }
}

template <class E>
static void launch_rot_e(const kd_rot_args& a, hipStream_t st) {
  if (a.inverse) launch_rot_d<E, true>(a, st);
  else launch_rot_d<E, false>(a, st);
}

int launch_hadamard(const kd_rot_args& a, hipStream_t st) {
  if (a.dtype == KD_BF16) launch_rot_e<BF16>(a, st);
  else if (a.dtype == KD_F16) launch_rot_e<F16>(a, st);
  else launch_rot_e<F32>(a, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
