// Shared device helpers for the gfx950 attention kernels.
//
// Token mask codes (one uint32 per token, built by kd_mask.hip):
//   bit 0  P  is_prefix
//   bit 1  S  in_span
//   bit 2  M  MASKQ (span_id == -1, only when span_id is given)
//   bit 3  C  context  (= !P & !S & !M)
//   bits 4-7  A  accept mask: which key flag bits this token, as a QUERY, sees
//             unconditionally:  P|C -> {P},  S -> {C},  M -> {S, P}
//   bits 8-31 R  span group: 0, or 1 + first position of this token's span id
//             (only for tokens with S and span_id > 0)
// Tokens at or beyond seq_len = min(lens[b], T) get code 0 (see nothing, seen
// by nothing).  With these codes the 7-term rule of original_kernel.py:478-517
// becomes
//   allow(i, j) = (A_i & flags_j) | (C_i & C_j & i >= j) | (R_i != 0 & R_i == R_j)
// because prefix_to_prefix | context_to_prefix | maskq_to_cls are "key is P",
// span_to_context is "key is C", maskq_to_spans is "key is S", context_causal
// is the C&C&i>=j term and same_span is the R equality.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define KD_DEV __device__ __forceinline__

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

namespace kd {

enum : uint32_t { FLAG_P = 1u, FLAG_S = 2u, FLAG_M = 4u, FLAG_C = 8u };

KD_DEV bool allow(uint32_t qc, uint32_t kc, int i, int j) {
  return (((qc >> 4) & kc & 0xFu) != 0u) | (((qc & kc & FLAG_C) != 0u) & (i >= j)) |
         (((qc >> 8) != 0u) & ((qc >> 8) == (kc >> 8)));
}

// The 64-bit masks of a PARTIAL tile, built in the kernels from token codes
// with wave ballots (the rule of allow(), term for term; the plan keeps only
// codes, classes and lists).  Every lane of the wave must call them
// (uniform control flow): lane l supplies the code of the other side's token
// 64 tile + l, 0 past T or seq_len, which allows nothing.
//
// query_row_mask: bit j = allow(i, k0 + j) for this lane's query i (code qc)
// over keys k0 .. k0 + 63, kc = code of key k0 + lane.
KD_DEV uint64_t query_row_mask(uint32_t qc, int i, uint32_t kc, int k0) {
  const uint32_t A = (qc >> 4) & 15u;
  const uint64_t kp = __builtin_amdgcn_ballot_w64((kc & FLAG_P) != 0u);
  const uint64_t ks = __builtin_amdgcn_ballot_w64((kc & FLAG_S) != 0u);
  const uint64_t km = __builtin_amdgcn_ballot_w64((kc & FLAG_M) != 0u);
  const uint64_t kx = __builtin_amdgcn_ballot_w64((kc & FLAG_C) != 0u);
  uint64_t row = ((A & FLAG_P) ? kp : 0u) | ((A & FLAG_S) ? ks : 0u) | ((A & FLAG_M) ? km : 0u) |
                 ((A & FLAG_C) ? kx : 0u);
  if (qc & FLAG_C) {  // C & C & i >= j: keys k0 .. i
    const int d = i - k0;
    row |= kx & (d >= 63 ? ~uint64_t(0) : (d < 0 ? uint64_t(0) : (uint64_t(2) << d) - 1u));
  }
  // same span: R_i != 0 and R_j == R_i, one ballot per distinct R_j of the tile
  const uint32_t kr = kc >> 8, qr = qc >> 8;
  uint64_t todo = __builtin_amdgcn_ballot_w64(kr != 0u);
  while (todo != 0u) {  // uniform, at most 64 iterations
    const uint32_t v = uint32_t(__builtin_amdgcn_readlane(int(kr), int(__builtin_ctzll(todo))));
    const uint64_t same = __builtin_amdgcn_ballot_w64(kr == v);
    todo &= ~same;
    if (qr == v) row |= same;
  }
  return row;
}

// key_col_mask: bit r = allow(q0 + r, j) for this lane's key j (code kc) over
// queries q0 .. q0 + 63, qc = code of query q0 + lane.
KD_DEV uint64_t key_col_mask(uint32_t kc, int j, uint32_t qc, int q0) {
  const uint32_t A = (qc >> 4) & 15u;
  const uint64_t ap = __builtin_amdgcn_ballot_w64((A & FLAG_P) != 0u);
  const uint64_t as = __builtin_amdgcn_ballot_w64((A & FLAG_S) != 0u);
  const uint64_t am = __builtin_amdgcn_ballot_w64((A & FLAG_M) != 0u);
  const uint64_t ac = __builtin_amdgcn_ballot_w64((A & FLAG_C) != 0u);
  uint64_t col = ((kc & FLAG_P) ? ap : 0u) | ((kc & FLAG_S) ? as : 0u) | ((kc & FLAG_M) ? am : 0u) |
                 ((kc & FLAG_C) ? ac : 0u);
  const uint64_t qx = __builtin_amdgcn_ballot_w64((qc & FLAG_C) != 0u);
  if (kc & FLAG_C) {  // C & C & i >= j: queries j .. q0 + 63
    const int d = j - q0;
    col |= qx & (d <= 0 ? ~uint64_t(0) : (d > 63 ? uint64_t(0) : ~((uint64_t(1) << d) - 1u)));
  }
  const uint32_t kr = kc >> 8, qr = qc >> 8;
  uint64_t todo = __builtin_amdgcn_ballot_w64(qr != 0u);
  while (todo != 0u) {  // uniform, at most 64 iterations
    const uint32_t v = uint32_t(__builtin_amdgcn_readlane(int(qr), int(__builtin_ctzll(todo))));
    const uint64_t same = __builtin_amdgcn_ballot_w64(qr == v);
    todo &= ~same;
    if (kr == v) col |= same;
  }
  return col;
}

// s if bit `pos` of w is set, else -inf (v_bfe_i32 + v_bfi_b32).
KD_DEV float mask_bit(float s, uint32_t w, int pos) {
  const uint32_t m = uint32_t(__builtin_amdgcn_sbfe(int(w), pos, 1u));
  return __uint_as_float((__float_as_uint(s) & m) | (0xFF800000u & ~m));
}

// Element types -----------------------------------------------------------
struct BF16 {};
struct F16 {};
struct F32 {};  // fp32 operands (the vector-ALU kernels of kd_simt.hip)

template <class E> KD_DEV f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);
template <> KD_DEV f32x16 mfma32x32x16<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> KD_DEV f32x16 mfma32x32x16<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two fp32 -> packed pair of 16-bit values (round to nearest even).
template <class E> KD_DEV uint32_t pack2(float lo, float hi);
template <> KD_DEV uint32_t pack2<BF16>(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <> KD_DEV uint32_t pack2<F16>(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

template <class E> KD_DEV float to_f32(uint16_t bits);
template <> KD_DEV float to_f32<BF16>(uint16_t bits) { return __uint_as_float(uint32_t(bits) << 16); }
template <> KD_DEV float to_f32<F16>(uint16_t bits) {
  return float(__builtin_bit_cast(_Float16, bits));
}

// The rounding residual of a packed pair: with w = pack2<E>(lo, hi), returns
// pack2<E>(lo - lo_w, hi - hi_w) where lo_w, hi_w are w's two values, so the
// pair (w, residual) carries lo and hi to about twice the type's significant
// bits (w + residual, as two MFMAs into one fp32 accumulator).
template <class E> KD_DEV uint32_t pack2_residual(float lo, float hi, uint32_t w) {
  return pack2<E>(lo - to_f32<E>(uint16_t(w & 0xFFFFu)), hi - to_f32<E>(uint16_t(w >> 16)));
}
// The third part of a three-way split: with w = pack2<E>(lo, hi) and r =
// pack2_residual<E>(lo, hi, w), the 16-bit rounding of what w + r leave
// over (both subtractions are exact in fp32), so that w + r + the result
// carry lo and hi to about three times the type's significant bits.
template <class E> KD_DEV uint32_t pack2_residual2(float lo, float hi, uint32_t w, uint32_t r) {
  return pack2<E>(lo - to_f32<E>(uint16_t(w & 0xFFFFu)) - to_f32<E>(uint16_t(r & 0xFFFFu)),
                  hi - to_f32<E>(uint16_t(w >> 16)) - to_f32<E>(uint16_t(r >> 16)));
}
// Eight fp32 values as a 16-bit MFMA operand (u32x4), and their residual
template <class E> KD_DEV u32x4 pack8(const float* p) {
  return u32x4{pack2<E>(p[0], p[1]), pack2<E>(p[2], p[3]), pack2<E>(p[4], p[5]), pack2<E>(p[6], p[7])};
}
template <class E> KD_DEV u32x4 pack8_residual(const float* p, const u32x4& w) {
  return u32x4{pack2_residual<E>(p[0], p[1], w[0]), pack2_residual<E>(p[2], p[3], w[1]),
               pack2_residual<E>(p[4], p[5], w[2]), pack2_residual<E>(p[6], p[7], w[3])};
}
template <class E> KD_DEV u32x4 pack8_residual2(const float* p, const u32x4& w, const u32x4& r) {
  return u32x4{pack2_residual2<E>(p[0], p[1], w[0], r[0]), pack2_residual2<E>(p[2], p[3], w[1], r[1]),
               pack2_residual2<E>(p[4], p[5], w[2], r[2]), pack2_residual2<E>(p[6], p[7], w[3], r[3])};
}

// Row permutation used for the A operand of 32x32 MFMAs whose output feeds the
// next MFMA's B operand straight from registers.  The 32x32 f32 accumulator
// gives lane (h = lane/32, c = lane%32) the rows 8g + 4h + i (g, i in 0..3).
// Loading MFMA row rho from logical row sigma(rho) = rho with bits 2 and 3
// swapped makes accumulator register r hold logical row 16*(r/8) + 8h + r%8,
// i.e. registers 8t..8t+7 are exactly the 8 consecutive k-slots lane half h
// must supply for k-step t of the following 32x32x16 MFMA.
KD_DEV int sigma(int rho) { return (rho & ~12) | ((rho & 4) << 1) | ((rho & 8) >> 1); }


// Inclusive scan of one int per thread over the workgroup (up to 16 waves;
// s_warp: 16 ints of LDS).  Every thread must call it.
KD_DEV int block_scan(int v, int* s_warp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (lane == 63) s_warp[wave] = v;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += s_warp[w];
  __syncthreads();
  return v + base;
}

KD_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
KD_DEV float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace kd
