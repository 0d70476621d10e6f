// Backward of the hierarchical-mask flash attention on gfx950 MFMA.
//
// Algebra of original_kernel.py:1239-1335 (dQ) and :1425-1524 (dK/dV), with
// P recomputed from the saved base-2 LSE, Delta = rowsum(O * dO) (:695) and
// the tile map driving both loops.  Unlike the reference with causal=True
// (:1199-1207, :1366-1375) the loops visit EVERY non-empty tile, so the
// gradient is the true gradient of the forward's mask.
//
// Delta is formed from O + O_lo when the forward stored the rounding residual
// O_lo (a->o_lo), i.e. from O to ~16 significant bits: Delta feeds the
// cancellation dP - Delta, where the bf16 rounding of O alone costs about 1%
// RMS in dQ on peaked rows.
// Workspace: a->delta holds 2 * B*H*T floats, Delta followed by LSEb, a copy
// of the LSE with -inf (fully masked rows) replaced by +inf so that
// exp2(S c - LSEb) is 0 on such rows without a per-element test.
//
// dQ kernel: 4 waves x 32 query rows per workgroup, 64 keys per step:
//   S^T  = K Q^T,  dP^T = V dO^T          (A = K, V rows from LDS; B = Q, dO regs)
//   dS^T = P^T * (dP^T - Delta)            (per-lane Delta, LSE)
//   dQ^T += K^T dS^T                       (A = K^T read transposed from LDS)
// dK/dV kernel: 4 wave pairs x 32 keys per workgroup, 64 queries per step:
//   S = Q K^T,  dP = dO V^T                (A = Q, dO rows from LDS; B = K, V regs)
//   dV^T += dO^T P,  dK^T += Q^T dS        (A = dO^T, Q^T read transposed)
// with S/P/dV on one wave of a pair and dP/dS/dK (one tile behind) on the other.
// Both keep the accumulated gradient transposed in registers so the MFMA
// output of one product is the register-resident B operand of the next, and
// both stream their tiles global -> LDS with buffer_load ... lds into the
// swizzled layout of kd_tile.h (double buffered; dK/dV's Q triple buffered).
#include "kd_tile.h"

namespace kd {

// LDS operand reads run this many MFMA steps ahead of their use in the dQ and
// dK/dV products
constexpr int DQ_PF = 3;
constexpr int DKDV_PF = 3;

// The workspace holds -Delta per row (dK/dV starts its dP accumulators from
// it), then -LSE / c with c the score scale
// (sm_scale log2 e, times q_scale k_scale for fp8 scores) and -inf for fully
// masked rows.  The dK/dV kernel starts each S accumulator from it, so that
// its P = exp2(c (S - LSE / c)) is one multiply and one exp2, and the LSE
// values are read before the product instead of between the product and the
// exponentials.
KD_DEV float score_scale(const AttnArgs& a, int bh) {
  return a.sm_scale * 1.4426950408889634f * (a.q8 != nullptr ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
}
KD_DEV float lse_neg_scaled(const AttnArgs& a, int bh, float l) {
  return l == -__builtin_inff() ? -__builtin_inff() : -l * (1.f / score_scale(a, bh));
}

// ---------------------------------------------------------------- Delta ----
template <class E, int D>
__global__ __launch_bounds__(256) void k_delta(AttnArgs a) {
  constexpr int TPR = D / 8;        // threads per row, 8 elements each
  constexpr int RPB = 256 / TPR;    // rows per block
  const int tid = threadIdx.x, seg = tid % TPR;
  const int64_t row = int64_t(blockIdx.x) * RPB + tid / TPR;
  const int64_t nrows = int64_t(a.B) * a.H * a.T;
  float sum = 0.f;
  if (row < nrows) {
    const int t = int(row % a.T);
    const int bh = int(row / a.T);
    const int b = bh / a.H, h = bh % a.H;
    const uint16_t* op = static_cast<const uint16_t*>(a.o) + b * a.o_strides[0] + h * a.o_strides[1] +
                         t * a.o_strides[2] + seg * 8;
    const uint16_t* dp = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1] +
                         t * a.do_strides[2] + seg * 8;
    const u32x4 ov = *reinterpret_cast<const u32x4*>(op);
    const u32x4 dv = *reinterpret_cast<const u32x4*>(dp);
    // O's residual: 16-bit, or fp32 at precision KD_PREC_SPLIT3
    float lo[8] = {};
    if (a.o_lo != nullptr) {
      if (a.precision == KD_PREC_SPLIT3) {
        const float* l32 = static_cast<const float*>(a.o_lo) + row * D + seg * 8;
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(l32), x1 = *reinterpret_cast<const f32x4*>(l32 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) lo[i] = x0[i], lo[4 + i] = x1[i];
      } else {
        const u32x4 lv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.o_lo) + row * D + seg * 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) lo[2 * w] = to_f32<E>(uint16_t(lv[w] & 0xFFFFu)), lo[2 * w + 1] = to_f32<E>(uint16_t(lv[w] >> 16));
      }
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float o0 = to_f32<E>(uint16_t(ov[w] & 0xFFFFu)) + lo[2 * w];
      const float o1 = to_f32<E>(uint16_t(ov[w] >> 16)) + lo[2 * w + 1];
      sum += o0 * to_f32<E>(uint16_t(dv[w] & 0xFFFFu));
      sum += o1 * to_f32<E>(uint16_t(dv[w] >> 16));
    }
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (row < nrows && seg == 0) {
    a.delta[row] = -sum;
    a.delta[nrows + row] = lse_neg_scaled(a, int(row / a.T), a.lse[row]);
  }
}

// A transposed accumulator's rows times scale, as the 16-bit type; with glo
// also each value's rounding residual at the same offsets of glo (the
// caller's contiguous residual row), so that g + glo carries the fp32 value to
// about twice the type's significant bits
// dlim: columns from there on are not stored (head dims 16 and 32 on the
// D = 64 kernels).  lo32: glo holds fp32 residuals (precision KD_PREC_SPLIT3),
// so that g + glo is the fp32 value.
template <class E, int D>
KD_DEV void store_rows_T(uint16_t* g, const f32x16 (&acc)[D / 32], float scale, int hf, void* glo = nullptr,
                         int dlim = D, bool lo32 = false) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const int d0 = 32 * db + 8 * gg + 4 * hf;
      if (d0 >= dlim) continue;
      const float f[4] = {acc[db][4 * gg] * scale, acc[db][4 * gg + 1] * scale, acc[db][4 * gg + 2] * scale,
                          acc[db][4 * gg + 3] * scale};
      const u32x2 w = {pack2<E>(f[0], f[1]), pack2<E>(f[2], f[3])};
      *reinterpret_cast<u32x2*>(g + d0) = w;
      if (glo != nullptr && lo32)
        *reinterpret_cast<f32x4*>(static_cast<float*>(glo) + d0) =
            f32x4{f[0] - to_f32<E>(uint16_t(w[0] & 0xFFFFu)), f[1] - to_f32<E>(uint16_t(w[0] >> 16)),
                  f[2] - to_f32<E>(uint16_t(w[1] & 0xFFFFu)), f[3] - to_f32<E>(uint16_t(w[1] >> 16))};
      else if (glo != nullptr)
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(glo) + d0) =
            u32x2{pack2_residual<E>(f[0], f[1], w[0]), pack2_residual<E>(f[2], f[3], w[1])};
    }
  }
}

// The contiguous residual row [.., a.D] of element row `row` of a residual
// buffer (16-bit, or fp32 at precision KD_PREC_SPLIT3); NULL stays NULL
KD_DEV void* lo_row(void* base, int64_t row, int dim, bool lo32) {
  if (base == nullptr) return nullptr;
  return lo32 ? static_cast<void*>(static_cast<float*>(base) + row * dim)
              : static_cast<void*>(static_cast<uint16_t*>(base) + row * dim);
}

// The rows of a transposed accumulator times R^T, R = diag(s) H_D / sqrt(D)
// (the inverse of kd_hadamard's rotation), stored like store_rows_T: the
// Walsh-Hadamard butterflies over d in registers, then the signs and
// scale / sqrt(D).  Lane half hf holds d = 32 db + 8 gg + 4 hf + i in
// register r = 16 db + 4 gg + i of acc, so bits 0, 1, 3, 4, 5, 6 of d pair
// registers of the lane and bit 2 pairs the two lane halves.
template <class E, int D>
KD_DEV void store_rows_T_unrot(uint16_t* g, f32x16 (&acc)[D / 32], float scale, int hf, const float* signs) {
  constexpr int NR = D / 2;
#pragma unroll
  for (int bit = 1; bit < NR; bit <<= 1)
#pragma unroll
    for (int r = 0; r < NR; ++r)
      if (!(r & bit)) {
        const float x = acc[r >> 4][r & 15], y = acc[(r | bit) >> 4][(r | bit) & 15];
        acc[r >> 4][r & 15] = x + y;
        acc[(r | bit) >> 4][(r | bit) & 15] = x - y;
      }
#pragma unroll
  for (int r = 0; r < NR; ++r) {  // p[0]: the value of the hf = 0 lane, p[1]: of the hf = 1 lane
    const float x = acc[r >> 4][r & 15];
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    acc[r >> 4][r & 15] = hf ? __uint_as_float(p[0]) - __uint_as_float(p[1]) : __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  const float c = scale * (D == 256 ? 0.0625f : D == 128 ? 0.088388347648318440f : 0.125f);  // scale / sqrt(D)
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const int d0 = 32 * db + 8 * gg + 4 * hf;
      float f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = acc[db][4 * gg + i] * (signs[d0 + i] * c);
      const u32x2 w = {pack2<E>(f[0], f[1]), pack2<E>(f[2], f[3])};
      *reinterpret_cast<u32x2*>(g + d0) = w;
    }
  }
}

// Byte offsets of the transposed A-operand reads (tile^T, 32 columns x 16 rows
// per MFMA k-step) for this lane: [db][half], k-step ks adds ks * 16 rows.
template <int D>
KD_DEV void tr_addrs(int lane, int (&addr)[D / 32][2]) {
  using TL = Tile<D>;
  const int i = lane & 15, g = lane >> 4;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int r = 8 * (g >> 1) + 4 * half + (i >> 2);
      const int chunk = 4 * db + 2 * (g & 1) + ((i & 3) >> 1);
      addr[db][half] = TL::at(r, chunk) + 8 * (i & 1);
    }
}

// ------------------------------------------------------------------- dQ ----
// DH, D0: this launch accumulates dQ's columns [D0, D0 + DH) (D = 256 runs
// two launches of 128 columns, each recomputing S and dP, so that the dQ
// accumulators fit next to the operands of the full head dim)
// NSP: the parts dS enters dQ in (1, 2 or 3: parts_of the precision)
template <class E, int D, bool Q8, int NSP, int DH = D, int D0 = 0>
__global__ __launch_bounds__(256, D <= 128 ? 2 : 1) void k_dq(AttnArgs a, const uint32_t* __restrict__ codes,
                                               const uint32_t* __restrict__ list,
                                               const int32_t* __restrict__ count,
                                               const uint32_t* __restrict__ order, int nT, int nQB,
                                               bool fuse_delta) {
  constexpr bool SP = NSP >= 2, S3 = NSP == 3;
  using TL = Tile<D>;
  using SO = ScoreOp<E, D, Q8>;  // S^T = K Q^T (16-bit, or fp8 from the K8 tile)
  using TK8 = typename ScoreOp<E, D, true>::TL;
  // fp8 scores (Q8) take S from the K8 tile, so the 16-bit K tile feeds only
  // dQ^T += K^T dS^T, i.e. only this launch's columns [D0, D0 + DH): it is
  // loaded DH wide (KHALF), which keeps the d = 256 launch's two slots of K,
  // V and K8 within the LDS
  constexpr bool KHALF = Q8 && DH < D;
  using TLK = Tile<KHALF ? DH : D>;  // 16-bit K tiles
  constexpr int DS = D / 16, DB = DH / 32, NL = TL::LOADS_PER_WAVE, NLK = TLK::LOADS_PER_WAVE,
                NL8 = TK8::LOADS_PER_WAVE;
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][TLK::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][TL::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_k8[Q8 ? 2 : 1][Q8 ? TK8::BYTES : 16];
  // the 64 key codes of each step's tile (lane = key), from which PARTIAL
  // tiles build their row masks (query_row_mask), copied one step ahead by
  // wave 0 into one of two slots.  The fp8 variant's tiles fill the 80 KB
  // that two workgroups a CU allow: it loads the codes into a register one
  // step ahead instead (settled at the step's start, see settle)
  constexpr bool LDS_CODES = !Q8;
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[LDS_CODES ? 2 : 1][64];

  // the wave index through readfirstlane: uniform, so the role and slot
  // arithmetic derived from it stays scalar
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, hf = lane >> 5,
            c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int h = work / (a.B * nQB);  // head-major, then the plan's longest-first order
  const int item = int(order[work - h * (a.B * nQB)]);
  const int b = item / nQB, qblock = item - b * nQB, bh = b * H + h;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t qrb = uint32_t(a.q_strides[2]) * 2u, dorb = uint32_t(a.do_strides[2]) * 2u,
                 krb = uint32_t(a.k_strides[2]) * 2u, vrb = uint32_t(a.v_strides[2]) * 2u;
  const auto rs_q = make_rsrc(qg, uint32_t(T) * qrb);
  const auto rs_do = make_rsrc(dog, uint32_t(T) * dorb);
  const u32x4 rs_k = rsrc_words(kg, uint32_t(T) * krb);
  const u32x4 rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  const int64_t BHT = int64_t(a.B) * H * T;

  const int qrow = qblock * 128 + wave * 32 + c;
  const bool qvalid = qrow < T;
  SO so;  // B operand: this lane's query row (Q, or its fp8 copy)
  // bytes of a row of the 16-bit inputs: 2 D, or fewer for head dims 16 and
  // 32 on the D = 64 kernel, whose other columns are read as zeros
  const uint32_t dbytes = uint32_t(a.D) * 2u;
  if constexpr (Q8) so.load_b(make_rsrc(a.q8 + int64_t(bh) * T * D, uint32_t(T) * D), uint32_t(qrow) * D, hf);
  else so.load_b(rs_q, uint32_t(qrow) * qrb, hf, dbytes);
  u32x4 dof[DS];
#pragma unroll
  for (int st = 0; st < DS; ++st) {
    const uint32_t col = (16 * st + 8 * hf) * 2;
    dof[st] = buf_load16(rs_do, col_masked(uint32_t(qrow) * dorb + col, col, dbytes));
  }
  const float INF = __builtin_inff();
  float lse, delta;
  if (fuse_delta) {  // uniform: compute this row's Delta and LSE copy here, for the dK/dV kernel too
    // Delta = sum_d dO (O + O_lo) over this lane's 64 elements, then the other half-wave's
    const uint16_t* og = static_cast<const uint16_t*>(a.o) + b * a.o_strides[0] + h * a.o_strides[1];
    const uint32_t orb = uint32_t(a.o_strides[2]) * 2u;
    const auto rs_o = make_rsrc(og, uint32_t(T) * orb);
    // o_lo is contiguous [B, H, T, a.D] (fp32 with S3); without it the empty
    // resource reads zeros
    const uint32_t lsz = S3 ? 4u : 2u;  // bytes per residual element
    const uint8_t* lg = a.o_lo == nullptr ? nullptr
                                          : static_cast<const uint8_t*>(a.o_lo) + int64_t(bh) * T * a.D * lsz;
    const auto rs_lo = make_rsrc(lg, lg == nullptr ? 0u : uint32_t(T) * uint32_t(a.D) * lsz);
    float sum = 0.f;
#pragma unroll
    for (int st = 0; st < DS; ++st) {
      const uint32_t col = (16 * st + 8 * hf) * 2;
      const u32x4 ov = buf_load16(rs_o, col_masked(uint32_t(qrow) * orb + col, col, dbytes));
      float lo[8];
      if constexpr (S3) {
        const uint32_t l0 = uint32_t(qrow) * dbytes * 2u + col * 2u;
        const u32x4 x0 = buf_load16(rs_lo, col_masked(l0, col, dbytes));
        const u32x4 x1 = buf_load16(rs_lo, col_masked(l0 + 16u, col, dbytes));
#pragma unroll
        for (int i = 0; i < 4; ++i) lo[i] = __uint_as_float(x0[i]), lo[4 + i] = __uint_as_float(x1[i]);
      } else {
        const u32x4 lv = buf_load16(rs_lo, col_masked(uint32_t(qrow) * dbytes + col, col, dbytes));
#pragma unroll
        for (int w = 0; w < 4; ++w)
          lo[2 * w] = to_f32<E>(uint16_t(lv[w] & 0xFFFFu)), lo[2 * w + 1] = to_f32<E>(uint16_t(lv[w] >> 16));
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float o0 = to_f32<E>(uint16_t(ov[w] & 0xFFFFu)) + lo[2 * w];
        const float o1 = to_f32<E>(uint16_t(ov[w] >> 16)) + lo[2 * w + 1];
        sum += o0 * to_f32<E>(uint16_t(dof[st][w] & 0xFFFFu));
        sum += o1 * to_f32<E>(uint16_t(dof[st][w] >> 16));
      }
    }
    delta = xhalf_sum(sum);
    const float l = qvalid ? a.lse[int64_t(bh) * T + qrow] : -INF;
    lse = (l == -INF) ? INF : l;
    if (qvalid && hf == 0) {
      a.delta[int64_t(bh) * T + qrow] = -delta;
      a.delta[BHT + int64_t(bh) * T + qrow] = lse_neg_scaled(a, bh, l);
    }
  } else {
    const float l = qvalid ? a.lse[int64_t(bh) * T + qrow] : -INF;
    lse = (l == -INF) ? INF : l;  // exp2(S c - inf) = 0: fully masked rows get no gradient
    delta = qvalid ? -a.delta[int64_t(bh) * T + qrow] : 0.f;
  }
  // dP^T accumulators start from -Delta (every register of a lane holds its
  // query's value), so dS = P dP needs no subtraction per score
  f32x16 neg_delta;
#pragma unroll
  for (int r = 0; r < 16; ++r) neg_delta[r] = -delta;
  // this wave's rows lie in q-tile 2 qblock + member (the member's class per key tile)
  const int member = wave >> 1;
  // token codes of batch row b (reads past T return 0: allow nothing)
  const u32x4 rs_codes = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  const uint32_t* codes_b = codes + int64_t(b) * T;
  uint32_t qcode = qvalid ? codes_b[qrow] : 0u;

  const int lbase = item;  // b nQB + qblock
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  uint32_t koff[NLK], voff[NL], k8off[NL8];
  TLK::load_offsets(wave, lane, krb, koff, KHALF ? uint32_t(DH) * 2u : dbytes);
  TL::load_offsets(wave, lane, vrb, voff, dbytes);
  TK8::load_offsets(wave, lane, uint32_t(D), k8off);
  const u32x4 rs_k8 = rsrc_words(Q8 ? a.k8 + int64_t(bh) * T * D : nullptr, Q8 ? uint32_t(T) * D : 0u);
  // inline-asm copies (dma_b128): the compiler places no wait for them
  // before this step's LDS reads, so tile e+1 loads during all of step e
  auto load_tile = [&](int kt, int buf) {
    const uint32_t k0 = uint32_t(kt) * 64u;
    // (KHALF: the tile's columns start at D0 of the row)
    TLK::load_async(rs_k, k0 * krb + (KHALF ? uint32_t(D0) * 2u : 0u), koff, lds_addr(s_k[buf]), wave);
    TL::load_async(rs_v, k0 * vrb, voff, lds_addr(s_v[buf]), wave);
    if constexpr (Q8) TK8::load_async(rs_k8, k0 * uint32_t(D), k8off, lds_addr(s_k8[buf]), wave);
  };
  // tile e's key codes, copied one step ahead of their use into LDS (a
  // register load would be waited for by the compiler together with the tile
  // copies issued after it), or into a register in the fp8 variant
  uint32_t kc_reg = 0, kc_next = 0;
  auto load_codes = [&](int e, int slot) {  // slot = e & 1
    const uint32_t j = entry_tile(ent[e]) * 64u + uint32_t(lane_here());
    if constexpr (LDS_CODES) {
      if (wave == 0) dma_b32(rs_codes, j * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_kc[slot][0])))));
    } else {
      (e == 0 ? kc_reg : kc_next) = j < uint32_t(T) ? codes_b[j] : 0u;
    }
  };

  const int srow = sigma(c);
  so.init(srow, hf);
  int raddr[DS];
#pragma unroll
  for (int st = 0; st < DS; ++st) raddr[st] = TL::at(srow, 2 * st + hf);
  int taddr_all[D / 32][2];
  tr_addrs<D>(lane, taddr_all);
  int taddr[DB][2];  // the column blocks of this launch (KHALF: the DH-wide tile's own)
  if constexpr (KHALF) {
    tr_addrs<DH>(lane, taddr);
  } else {
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      taddr[db][0] = taddr_all[D0 / 32 + db][0];
      taddr[db][1] = taddr_all[D0 / 32 + db][1];
    }
  }

  // the fp8 product carries the dequantisation scales of Q and K
  const float sl2 = a.sm_scale * 1.4426950408889634f * (Q8 ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  if (n > 0) {
    load_tile(int(entry_tile(ent[0])), 0);
    load_codes(0, 0);
  }
  // every register load of the prologue is complete here: the compiler's
  // waits for them fall here, none later in the loop (see settle)
  wait_vmem();
  so.settle();
#pragma unroll
  for (int st = 0; st < DS; ++st) settle(dof[st]);
  settle(lse);
  settle(delta);
  settle(qcode);

  // One step per key tile; unrolled by two so that the buffer of each step is
  // a constant and every LDS address is a fixed register plus an immediate.
  auto step = [&](const int e, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;  // == e & 1
    const uint32_t cur = ent[e];
    wait_vmem();
    if constexpr (!LDS_CODES) settle(kc_reg);
    barrier_raw();  // tile e (and its key codes) landed for every wave; every wave is done with tile e-1
    if (e + 1 < n) {
      load_tile(int(entry_tile(ent[e + 1])), buf ^ 1);
      load_codes(e + 1, buf ^ 1);
    }
    const uint8_t* kt = s_k[buf];
    const uint8_t* vt = s_v[buf];

    // the row mask is formed first: LDS reads cannot cross the products'
    // scheduling fences, and the mask must not hold back the softmax below
    const uint32_t mcls = entry_class(cur, member);
    uint64_t rowbits = 0;  // EMPTY: nothing allowed
    if (mcls == TILE_PARTIAL) {  // wave-uniform
      const int l = lane_here();  // (lane-derived values are recomputed here, not kept live)
      rowbits = query_row_mask(qcode, qblock * 128 + wave * 32 + (l & 31),
                               LDS_CODES ? s_kc[LDS_CODES ? buf : 0][l] : kc_reg, int(entry_tile(cur)) * 64);
    }

    // S^T = K Q^T and dP^T = V dO^T; A operands (K / K8 and V rows) are read
    // DQ_PF steps ahead of their MFMAs, steps i: kb = i & 1, st = i >> 1; the
    // sched_barriers keep LDS reads and MFMAs in that order
    f32x16 s[2], dp[2];
    {
      const uint8_t* st_tile = Q8 ? s_k8[Q8 ? buf : 0] : kt;
      constexpr int NS = 2 * SO::NK, PF = DQ_PF < NS ? DQ_PF : NS;
      typename SO::A av[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) av[i] = so.read_a(st_tile, i & 1, i >> 1);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        __builtin_amdgcn_sched_barrier(0x406);
        s[i & 1] = so.mma_a(av[i % PF], i >> 1, (i >> 1) == 0 ? f32x16{} : s[i & 1]);
        if (i + PF < NS) av[i % PF] = so.read_a(st_tile, (i + PF) & 1, (i + PF) >> 1);
      }
      __builtin_amdgcn_sched_barrier(0x406);
    }
    if (mcls != TILE_FULL) {  // wave-uniform.  Register r of s[kb] holds key 32 kb + 16 (r / 8) + 8 hf + r % 8
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const uint32_t w = uint32_t(rowbits >> (32 * kb)) >> (8 * hf);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = mask_bit(s[kb][r], w, 16 * (r >> 3) + (r & 7));
      }
    }
    // dP^T, started from -Delta, with P = exp2(S c - LSE) computed in place
    // between its MFMAs: EPI exponentials after each MFMA, held there by
    // fences that only scalar work may cross (left free, the scheduler puts
    // all of them ahead of the first dP MFMA)
    {
      constexpr int NS = 2 * DS, PF = DQ_PF;
      constexpr int EPI = 32 / NS;  // exponentials per dP step
      auto read = [&](int i) {
        return *reinterpret_cast<const u32x4*>(vt + raddr[i >> 1] + (i & 1) * 32 * TL::ROWB);
      };
      u32x4 av[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        __builtin_amdgcn_sched_barrier(0x4);
        dp[i & 1] = mfma32x32x16<E>(av[i % PF], dof[i >> 1], (i >> 1) == 0 ? neg_delta : dp[i & 1]);
        if (i + PF < NS) av[i % PF] = read(i + PF);
#pragma unroll
        for (int u = 0; u < EPI; ++u) {
          const int kb = i & 1, r = EPI * (i >> 1) + u;
          s[kb][r] = fast_exp2(__builtin_fmaf(s[kb][r], sl2, -lse));
        }
      }
      __builtin_amdgcn_sched_barrier(0x4);
    }
    // dS packed for the MFMA and, with SP, its rounding residual: dQ takes
    // dS to ~16 significant bits as two products (with S3, ~24 as three)
    u32x4 dsb[2][2];
    u32x4 dsl[SP ? 2 : 1][2];
    u32x4 dsm[S3 ? 2 : 1][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) ds[r] = s[kb][r] * dp[kb][r];  // dp = dP - Delta
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        dsb[kb][t] = pack8<E>(ds + 8 * t);
        if constexpr (SP) dsl[kb][t] = pack8_residual<E>(ds + 8 * t, dsb[kb][t]);
        if constexpr (S3) dsm[kb][t] = pack8_residual2<E>(ds + 8 * t, dsb[kb][t], dsl[kb][t]);
      }
    }
    // dQ^T += K^T dS^T, K^T read transposed DQ_PF steps ahead (steps: t4 = i / DB, db = i % DB)
    {
      constexpr int NS = 4 * DB, PF = DQ_PF;
      auto read = [&](int i) {
        const int t4 = i / DB, db = i % DB;
        const u32x2 lo = ds_read_tr16(kt + taddr[db][0] + t4 * 16 * TLK::ROWB);
        const u32x2 hi = ds_read_tr16(kt + taddr[db][1] + t4 * 16 * TLK::ROWB);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 av[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int t4 = i / DB, db = i % DB;
        __builtin_amdgcn_sched_barrier(0x406);
        acc[db] = mfma32x32x16<E>(av[i % PF], dsb[t4 >> 1][t4 & 1], acc[db]);
        if constexpr (SP) acc[db] = mfma32x32x16<E>(av[i % PF], dsl[t4 >> 1][t4 & 1], acc[db]);
        if constexpr (S3) acc[db] = mfma32x32x16<E>(av[i % PF], dsm[S3 ? t4 >> 1 : 0][t4 & 1], acc[db]);
        if (i + PF < NS) av[i % PF] = read(i + PF);
      }
      __builtin_amdgcn_sched_barrier(0x406);
    }
    if constexpr (!LDS_CODES) kc_reg = kc_next;
  };
  for (int e = 0; e < n; e += 2) {
    step(e, std::integral_constant<int, 0>{});
    if (e + 1 < n) step(e + 1, std::integral_constant<int, 1>{});
  }

  if (qvalid) {
    uint16_t* g = static_cast<uint16_t*>(a.dq) + b * a.dq_strides[0] + h * a.dq_strides[1] + qrow * a.dq_strides[2];
    void* glo = lo_row(a.dq_lo, (int64_t(b) * a.H + h) * a.T + qrow, a.D, S3);
    if constexpr (DH == D) {
      if (a.dqk_signs != nullptr) store_rows_T_unrot<E, D>(g, acc, a.sm_scale, hf, a.dqk_signs);
      else store_rows_T<E, D>(g, acc, a.sm_scale, hf, glo, a.D, S3);
    } else {  // (no dqk_signs at split widths)
      void* glo_h = glo == nullptr ? nullptr : static_cast<void*>(static_cast<uint8_t*>(glo) + D0 * (S3 ? 4 : 2));
      store_rows_T<E, DH>(g + D0, acc, a.sm_scale, hf, glo_h, DH, S3);
    }
  }
}

// ---------------------------------------------------------------- dK/dV ----
// 8 waves per workgroup = 4 pairs, one pair per 32 keys (128 keys in all).
// The two waves of a pair split the work of their keys by role:
//   role 0 ("P wave"):  S = Q K^T, P = exp2(S c - LSE)   -> dV^T += dO^T P
//   role 1 ("dS wave"): dP = dO V^T, dS = P (dP - Delta) -> dK^T += Q^T dS
// P goes from the P wave to the dS wave through LDS (bf16, as the MFMA takes
// it), lane to lane: both waves hold the same MFMA output layout.  Each wave
// keeps one B operand (K or V) and one accumulator (dV^T or dK^T) in
// registers, so a pair needs about half the registers of one wave doing all
// four products; the pair shares a SIMD (waves w and w + 4).
// The dS wave runs one query tile behind: in step e the P wave handles tile
// e while the dS wave computes dP of tile e and finishes dS / dK of tile
// e - 1 with the P written in step e - 1.  So one barrier per step orders
// everything (tile e landed, P(e-1) written, P(e-2) and tile e-2 released),
// at the price of a third Q buffer (dK reads Q of tile e - 1).
// NSP: the parts P and dS enter dV and dK in (1, 2 or 3: parts_of the precision)
template <class E, int D, bool Q8, int NSP>
__global__ __launch_bounds__(512, 1) void k_dkdv(AttnArgs a, const uint32_t* __restrict__ codes,
                                                 const uint32_t* __restrict__ list,
                                                 const int32_t* __restrict__ count,
                                                 const uint32_t* __restrict__ order, int nT, int nKB) {
  constexpr bool SP = NSP >= 2, S3 = NSP == 3;
  constexpr int NW = 8;
  using TL = Tile<D, NW>;
  using TQ8 = Tile<Q8 ? D / 2 : D, 4>;  // fp8 Q tiles (D bytes a row): their layout (TC8 copies them)
  constexpr int DS = D / 16, DB = D / 32;
  // Tiles are loaded PD steps ahead: 2, or 1 where the fp8 variant's Q8
  // tiles or SP's fp32 P exchange take the LDS.  Slot counts follow from who
  // reads what when: in step e the P waves read Q(e) (fp8: Q8(e)), dO(e),
  // LSE(e); the dS waves dO(e), Q(e-1), Delta(e-1); a load issued in step e
  // must not overwrite any of those.  The fp8 variant's 16-bit Q tile feeds
  // only the dK product, one step later, so its copy of tile e is issued in
  // step e itself, into one of two slots.
  constexpr int PD = (Q8 || SP) ? 1 : 2, NQ = Q8 ? 2 : PD + 2, NDO = PD + 1, NLS = PD + 1, NDL = PD + 2;
  __shared__ __attribute__((aligned(1024))) uint8_t s_q[NQ][TL::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_q8[Q8 ? NDO : 1][Q8 ? TQ8::BYTES : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t s_do[NDO][TL::BYTES];
  // P from the P wave to the dS wave, [e % 2][pair][k-step][lane]: packed
  // 16-bit P, or with SP the fp32 P (two u32x4 per k-step), so that dS = P (dP
  // - Delta) keeps P's full precision
  __shared__ __attribute__((aligned(1024))) u32x4 s_p[2][4][SP ? 8 : 4][64];
  __shared__ __attribute__((aligned(256))) float s_lse[NLS][64];
  __shared__ __attribute__((aligned(256))) float s_delta[NDL][64];
  // the 64 query codes of each step's q-tile (lane = query), from which the P
  // waves build a PARTIAL tile's column masks (key_col_mask); copied with the tile
  __shared__ __attribute__((aligned(256))) uint32_t s_qc[NLS][64];

  // (the wave index stays a vector value here: made uniform, the two roles'
  // registers are allocated apart and the kernel spills)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, c = lane & 31;
  const int pair = wave & 3, role = wave >> 2;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int h = work / (a.B * nKB);  // head-major, then the plan's longest-first dK/dV order
  const int item = int(order[work - h * (a.B * nKB)]);
  const int b = item / nKB, kblock = item - b * nKB, bh = b * H + h;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t qrb = uint32_t(a.q_strides[2]) * 2u, dorb = uint32_t(a.do_strides[2]) * 2u,
                 krb = uint32_t(a.k_strides[2]) * 2u, vrb = uint32_t(a.v_strides[2]) * 2u;
  const u32x4 rs_q = rsrc_words(qg, uint32_t(T) * qrb);
  const u32x4 rs_do = rsrc_words(dog, uint32_t(T) * dorb);
  const int64_t BHT = int64_t(a.B) * H * T;
  const u32x4 rs_lse = rsrc_words(a.delta + BHT + int64_t(bh) * T, uint32_t(T) * 4u);
  const u32x4 rs_dl = rsrc_words(a.delta + int64_t(bh) * T, uint32_t(T) * 4u);

  // this lane's key and its B operand: K for the P wave, V for the dS wave
  const int krow = kblock * 128 + pair * 32 + c;
  const bool kvalid = krow < T;
  u32x4 bf[DS];
  if (Q8 && role == 0) {
    // fp8: the P waves' B operand is this lane's row of K8; k-step st (64
    // bytes) takes bytes 64 st + 32 hf .. + 31, kept in bf[2 st], bf[2 st + 1]
    const auto rs8 = make_rsrc(a.k8 + int64_t(bh) * T * D, uint32_t(T) * D);
#pragma unroll
    for (int st = 0; st < D / 64; ++st) {
      bf[2 * st] = buf_load16(rs8, uint32_t(krow) * D + 64 * st + 32 * hf);
      bf[2 * st + 1] = buf_load16(rs8, uint32_t(krow) * D + 64 * st + 32 * hf + 16);
    }
  } else {
    // (a uniform role for the select: a per-lane buffer resource would need a readfirstlane loop per load)
    const bool p_wave = __builtin_amdgcn_readfirstlane(role) == 0;
    const auto rs_b = p_wave ? make_rsrc(kg, uint32_t(T) * krb) : make_rsrc(vg, uint32_t(T) * vrb);
    const uint32_t brb = role == 0 ? krb : vrb;
#pragma unroll
    for (int st = 0; st < DS; ++st) bf[st] = buf_load16(rs_b, uint32_t(krow) * brb + (16 * st + 8 * hf) * 2);
  }
  // this pair's keys lie in k-tile 2 kblock + member (the member's class per
  // q-tile); a PARTIAL tile's column masks, per key, come from the codes of
  // the key and of the q-tile's queries (reads past T return 0: allow nothing)
  const int member = pair >> 1;
  const u32x4 rs_codes = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  uint32_t kcode = kvalid ? codes[int64_t(b) * T + krow] : 0u;

  const int lbase = b * nKB + kblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  // The P waves make every copy (the four of them share each tile): the dS
  // waves carry the longer chain of a step, the P waves wait for them at the
  // barrier, so the copies' issue time is taken from the P waves' slack.
  // The per-lane copy offsets are recomputed at each copy from the lane id
  // (lane_here: not hoisted), which costs a few VALU instructions of the P
  // waves' slack instead of registers held across the loop.
  using TC = Tile<D, 4>;
  using TC8 = Tile<Q8 ? D / 2 : D, 4>;
  const u32x4 rs_q8 = rsrc_words(Q8 ? a.q8 + int64_t(bh) * T * D : nullptr, Q8 ? uint32_t(T) * D : 0u);
  // Tile e's copies, all inline asm (dma_b128 / dma_b32: the compiler places
  // no waits for them, so they stay in flight until wait_tile): per P wave
  // 2 TC::LOADS_PER_WAVE tile loads (fp8: Q8 and dO), then LSE (wave 1),
  // Delta (wave 2) and the query codes (wave 3), one load each.
  // Slots of tile e: e % NQ, e % NDO (Q8 tiles too), e % NLS (LSE, masks),
  // e % NDL; the loop keeps them as wrapping counters (uniform, no division).
  struct Slots { int q, d, ls, dl; };
  auto wrap = [](int x, int m) { return x >= m ? x - m : x; };
  auto ahead = [&](const Slots& s, int k) {  // slots of tile e + k (k < every slot count)
    return Slots{wrap(s.q + k, NQ), wrap(s.d + k, NDO), wrap(s.ls + k, NLS), wrap(s.dl + k, NDL)};
  };
  const bool copier = __builtin_amdgcn_readfirstlane(role) == 0;  // a P wave
  const int wave_u = __builtin_amdgcn_readfirstlane(wave), pair_u = wave_u & 3;
  auto load_tile = [&](uint32_t en, const Slots& sl) {  // en: the tile's list entry
    if (!copier) return;
    const uint32_t q0 = entry_tile(en) * 64u;
    const int ln = lane_here();
    const uint32_t lrow = TC::lane_row(pair_u, ln), c16 = TC::lane_chunk16(pair_u, ln);
    if constexpr (!Q8) TC::load_async_rows(rs_q, q0 * qrb, lrow * qrb, c16, qrb, lds_addr(s_q[sl.q]), pair_u);
    TC::load_async_rows(rs_do, q0 * dorb, lrow * dorb, c16, dorb, lds_addr(s_do[sl.d]), pair_u);
    if constexpr (Q8)
      TC8::load_async_rows(rs_q8, q0 * uint32_t(D), TC8::lane_row(pair_u, ln) * uint32_t(D),
                           TC8::lane_chunk16(pair_u, ln), uint32_t(D), lds_addr(s_q8[Q8 ? sl.d : 0]), pair_u);
    if (wave_u == 1)
      dma_b32(rs_lse, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_lse[sl.ls][0])))));
    else if (wave_u == 2)
      dma_b32(rs_dl, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_delta[sl.dl][0])))));
    else if (wave_u == 3)
      dma_b32(rs_codes, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_qc[sl.ls][0])))));
  };
  // fp8: the 16-bit Q tile of tile e (the dK product's operand in step e + 1)
  auto load_q16 = [&](uint32_t en, const Slots& sl) {
    if (!copier) return;
    const uint32_t q0 = entry_tile(en) * 64u;
    const int ln = lane_here();
    TC::load_async_rows(rs_q, q0 * qrb, TC::lane_row(pair_u, ln) * qrb, TC::lane_chunk16(pair_u, ln), qrb,
                        lds_addr(s_q[sl.q]), pair_u);
  };
  // Wait until tile e's loads (and older ones) have landed while tile e+1's,
  // issued last, may still be in flight: vector memory loads retire in order.
  // Waves 1, 2 and 3 issue one more load per tile (LSE, Delta, query codes);
  // the dS waves issue none.  Only used with PD = 2, i.e. neither fp8 nor SP.
  constexpr int NTL = 2 * TC::LOADS_PER_WAVE;
  auto wait_tile = [&](bool next_in_flight) {
    if (!next_in_flight || !copier) wait_vmem();
    else if (wave_u != 0) wait_vmem_n<NTL + 1>();
    else wait_vmem_n<NTL>();
  };

  const int srow = sigma(c);
  int raddr[DS];
#pragma unroll
  for (int st = 0; st < DS; ++st) raddr[st] = TL::at(srow, 2 * st + hf);
  int taddr[DB][2];
  tr_addrs<D>(lane, taddr);

  // the fp8 product carries the dequantisation scales of Q and K
  const float sl2 = a.sm_scale * 1.4426950408889634f * (Q8 ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
  f32x16 acc[DB];  // dV^T (role 0) or dK^T (role 1)
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  // Both products below read their A operands from LDS DKDV_PF steps ahead of
  // the MFMA that uses them; the sched_barriers keep LDS reads and MFMAs in
  // that order (VALU and SALU work may move across), which also bounds the
  // registers held by operands in flight.
  constexpr int PF = DKDV_PF;
  // acc^T += A^T bop over the 64 queries of a tile (k-steps k4 = 2 qb + t),
  // A^T read transposed from tile `at`; steps i = 4 k4 ... ordered (k4, db)
  // With SP, bopl holds the residual of bop and enters the same accumulator
  // through a second MFMA on the same A operand; with S3 bopm a third part.
  auto accumulate = [&](const uint8_t* at_g, const u32x4 (&bop)[2][2], const u32x4 (&bopl)[2][2],
                        const u32x4 (&bopm)[2][2]) {
    lds_u8* at = to_lds(at_g);
    constexpr int NS = 4 * DB;
    lds_u8* pa[DB][2];  // one address per (db, half); the k-step offsets are immediates
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      pa[db][0] = at + taddr[db][0];
      pa[db][1] = at + taddr[db][1];
    }
    auto read = [&](int i) {
      const int k4 = i / DB, db = i % DB, off = k4 * 16 * TL::ROWB;
      const u32x2 lo = ds_read_tr16(pa[db][0] + off);
      const u32x2 hi = ds_read_tr16(pa[db][1] + off);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    u32x4 av[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int k4 = i / DB, db = i % DB;
      __builtin_amdgcn_sched_barrier(0x406);
      acc[db] = mfma32x32x16<E>(av[i % PF], bop[k4 >> 1][k4 & 1], acc[db]);
      if constexpr (SP) acc[db] = mfma32x32x16<E>(av[i % PF], bopl[k4 >> 1][k4 & 1], acc[db]);
      if constexpr (S3) acc[db] = mfma32x32x16<E>(av[i % PF], bopm[k4 >> 1][k4 & 1], acc[db]);
      if (i + PF < NS) av[i % PF] = read(i + PF);
    }
    __builtin_amdgcn_sched_barrier(0x406);
  };
  // x[qb] += (rows of tile `ar`) B^T; register r of x[qb] holds query
  // 32 qb + 16 (r / 8) + 8 hf + r % 8 of this lane's key; steps i = (st, qb)
  // from_x: accumulate onto x's current content instead of zero
  auto rows_times_b = [&](const uint8_t* ar_g, f32x16 (&x)[2], bool from_x) {
    lds_u8* ar = to_lds(ar_g);
    constexpr int NS = 2 * DS;
    lds_u8* pr[DS];  // one address per k-step; the 32-row offset is an immediate
#pragma unroll
    for (int st = 0; st < DS; ++st) pr[st] = ar + raddr[st];
    auto read = [&](int i) { return ds_read16(pr[i >> 1] + (i & 1) * 32 * TL::ROWB); };
    u32x4 av[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int st = i >> 1, qb = i & 1;
      __builtin_amdgcn_sched_barrier(0x406);
      x[qb] = mfma32x32x16<E>(av[i % PF], bf[st], (st == 0 && !from_x) ? f32x16{} : x[qb]);
      if (i + PF < NS) av[i % PF] = read(i + PF);
    }
    __builtin_amdgcn_sched_barrier(0x406);
  };

  // list entries e .. e + PD - 1 at the start of step e, carried in SGPRs,
  // and en_next = entry e + PD (the tile step e copies), loaded at the end of
  // step e - 1: the P waves' class of tile e is not re-read from memory
  // inside the products, where a scalar load in flight would make every LDS
  // wait there wait for all outstanding LDS reads (scalar loads complete out
  // of order)
  uint32_t pend[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i) pend[i] = i < n ? ent[i] : 0u;
  Slots sl{0, 0, 0, 0};  // slots of tile e (e = 0 here)
  if (n > 0) load_tile(pend[0], sl);
  // the B operand's register loads are complete here: the compiler's wait
  // for them falls here, not at their first use (where it would also wait
  // for the copies of tile 1)
  wait_vmem();
#pragma unroll
  for (int st = 0; st < DS; ++st) settle(bf[st]);
  settle(kcode);
  if (PD > 1 && n > 1) load_tile(pend[PD > 1 ? 1 : 0], ahead(sl, 1));
  // S of tile e (P waves), or dP of tile e carried into step e + 1 (dS
  // waves): one register set for both roles
  f32x16 x[2] = {f32x16{}, f32x16{}};

  uint32_t en_next = PD < n ? ent[PD] : 0u;
  for (int e = 0; e <= n; ++e) {
    // tiles up to e landed (tile e + PD - 1 may be in flight when PD = 2)
    wait_tile(PD == 2 && e + 1 < n);
    barrier_lds();  // tile e landed, P(e-1) written; P(e-2) and the slots of tile e+PD released
    uint32_t en = pend[0];  // entry of tile e (e < n)
    asm volatile("" : "+s"(en));
    const uint32_t en_pd = en_next;  // entry of tile e + PD (loaded in step e - 1)
#pragma unroll
    for (int i = 0; i + 1 < PD; ++i) pend[i] = pend[i + 1];
    pend[PD - 1] = en_pd;
    const int pb = e & 1;
    if (role == 0) {
      if (e < n) {
        // S starts from -LSE / c of its query (register r of x[qb]: query
        // 32 qb + 16 (r / 8) + 8 hf + r % 8), so that P = exp2(c x)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int ql = 32 * qb + 16 * t + 8 * hf;
            const f32x4 l0 = *reinterpret_cast<const f32x4*>(&s_lse[sl.ls][ql]);
            const f32x4 l1 = *reinterpret_cast<const f32x4*>(&s_lse[sl.ls][ql + 4]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              x[qb][8 * t + j] = l0[j];
              x[qb][8 * t + 4 + j] = l1[j];
            }
          }
        if constexpr (Q8) {  // S = Q8 K8^T on the fp8 MFMA; A = Q8 rows, 32 bytes per lane and k-step
          const uint8_t* t8 = s_q8[Q8 ? sl.d : 0];
#pragma unroll
          for (int st = 0; st < D / 64; ++st) {
            const int a0 = TQ8::at(srow, 4 * st + 2 * hf), a1 = TQ8::at(srow, 4 * st + 2 * hf + 1);
            const i32x8 bv = {int(bf[2 * st][0]), int(bf[2 * st][1]), int(bf[2 * st][2]), int(bf[2 * st][3]),
                              int(bf[2 * st + 1][0]), int(bf[2 * st + 1][1]), int(bf[2 * st + 1][2]),
                              int(bf[2 * st + 1][3])};
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              const u32x4 lo = *reinterpret_cast<const u32x4*>(t8 + a0 + qb * 32 * TQ8::ROWB);
              const u32x4 hi = *reinterpret_cast<const u32x4*>(t8 + a1 + qb * 32 * TQ8::ROWB);
              const i32x8 av = {int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]),
                                int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
              x[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, x[qb], 0, 0, 0, 127, 0, 127);
            }
          }
        } else {
          rows_times_b(s_q[sl.q], x, true);
        }
        const uint32_t mcls = entry_class(en, member);
        if (mcls != TILE_FULL) {  // wave-uniform
          const uint64_t colbits = mcls == TILE_PARTIAL  // EMPTY: nothing allowed
                                       ? key_col_mask(kcode, krow, s_qc[sl.ls][lane_here()], int(entry_tile(en)) * 64)
                                       : 0u;
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            const uint32_t w = uint32_t(colbits >> (32 * qb)) >> (8 * hf);
#pragma unroll
            for (int r = 0; r < 16; ++r) x[qb][r] = mask_bit(x[qb][r], w, 16 * (r >> 3) + (r & 7));
          }
        }
        // this step's copies, after S (P waves only): tile e + PD into the
        // slots the barrier released, and for fp8 the 16-bit Q of tile e,
        // which the dS waves read in step e + 1
        if (e + PD < n) load_tile(en_pd, ahead(sl, PD));
        if constexpr (Q8) load_q16(en, sl);
        u32x4 bop[2][2];                // packed P: B operand of k-step 2 qb + t
        u32x4 bopl[2][2];               // SP: its rounding residual (unused otherwise)
        u32x4 bopm[2][2];               // S3: its third part (unused otherwise)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            float p[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) p[j] = fast_exp2(x[qb][8 * t + j] * sl2);
            bop[qb][t] = pack8<E>(p);
            if constexpr (SP) {
              bopl[qb][t] = pack8_residual<E>(p, bop[qb][t]);
              if constexpr (S3) bopm[qb][t] = pack8_residual2<E>(p, bop[qb][t], bopl[qb][t]);
              // the fp32 P for the dS wave, stored as it is formed (holding
              // it across the dV MFMAs would take 32 more registers)
              s_p[pb][pair][2 * (2 * qb + t)][lane] = u32x4{__float_as_uint(p[0]), __float_as_uint(p[1]),
                                                            __float_as_uint(p[2]), __float_as_uint(p[3])};
              s_p[pb][pair][2 * (2 * qb + t) + 1][lane] = u32x4{__float_as_uint(p[4]), __float_as_uint(p[5]),
                                                                __float_as_uint(p[6]), __float_as_uint(p[7])};
            }
          }
        accumulate(s_do[sl.d], bop, bopl, bopm);  // dV^T += dO^T P
        // 16-bit P for the dS wave (read after the next barrier).  Written
        // after the MFMAs: LDS stores may not cross the product's scheduling
        // fences, so stores placed before it would hold all of P's VALU work
        // ahead of the first MFMA.
        if constexpr (!SP) {
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int t = 0; t < 2; ++t) s_p[pb][pair][2 * qb + t][lane] = bop[qb][t];
        }
      }
    } else {
      if (e >= 1) {  // dS and dK of tile e - 1
        const int qprev = wrap(sl.q + NQ - 1, NQ);
        u32x4 dsb[2][2];
        u32x4 dsl[2][2];  // SP: dS's rounding residual (unused otherwise)
        u32x4 dsm[2][2];  // S3: its third part (unused otherwise)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            float ds[8];
            if constexpr (SP) {
              const u32x4 p0 = s_p[pb ^ 1][pair][2 * (2 * qb + t)][lane];
              const u32x4 p1 = s_p[pb ^ 1][pair][2 * (2 * qb + t) + 1][lane];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                ds[j] = __uint_as_float(p0[j]) * x[qb][8 * t + j];  // x = dP - Delta
                ds[4 + j] = __uint_as_float(p1[j]) * x[qb][8 * t + 4 + j];
              }
            } else {
              const u32x4 pw = s_p[pb ^ 1][pair][2 * qb + t][lane];
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                const uint32_t w = pw[j >> 1];
                const float p = to_f32<E>(uint16_t((j & 1) ? (w >> 16) : (w & 0xFFFFu)));
                ds[j] = p * x[qb][8 * t + j];  // x = dP - Delta (the product started from -Delta)
              }
            }
            dsb[qb][t] = pack8<E>(ds);
            if constexpr (SP) dsl[qb][t] = pack8_residual<E>(ds, dsb[qb][t]);
            if constexpr (S3) dsm[qb][t] = pack8_residual2<E>(ds, dsb[qb][t], dsl[qb][t]);
          }
        accumulate(s_q[qprev], dsb, dsl, dsm);  // dK^T += Q^T dS
      }
      if (e < n) {  // dP of tile e, started from -Delta of its query (register layout as for S)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int ql = 32 * qb + 16 * t + 8 * hf;
            const f32x4 d0 = *reinterpret_cast<const f32x4*>(&s_delta[sl.dl][ql]);
            const f32x4 d1 = *reinterpret_cast<const f32x4*>(&s_delta[sl.dl][ql + 4]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              x[qb][8 * t + j] = d0[j];
              x[qb][8 * t + 4 + j] = d1[j];
            }
          }
        rows_times_b(s_do[sl.d], x, true);
      }
    }
    // the entry of the tile the next step copies, loaded by the P waves after
    // their products (a scalar load in flight would make every LDS wait in
    // them wait for all outstanding LDS reads; here it completes while the
    // P waves wait at the barrier)
    __builtin_amdgcn_sched_barrier(0);
    if (copier) en_next = e + 1 + PD < n ? ent[e + 1 + PD] : 0u;
    sl = ahead(sl, 1);
  }

  if (kvalid) {
    uint16_t* g = role == 0
        ? static_cast<uint16_t*>(a.dv) + b * a.dv_strides[0] + h * a.dv_strides[1] + krow * a.dv_strides[2]
        : static_cast<uint16_t*>(a.dk) + b * a.dk_strides[0] + h * a.dk_strides[1] + krow * a.dk_strides[2];
    void* glo = lo_row(role == 0 ? a.dv_lo : a.dk_lo, (int64_t(b) * H + h) * T + krow, D, S3);
    if (__builtin_amdgcn_readfirstlane(role) == 1 && a.dqk_signs != nullptr)  // dK, rotated back
      store_rows_T_unrot<E, D>(g, acc, a.sm_scale, hf, a.dqk_signs);
    else
      store_rows_T<E, D>(g, acc, role == 0 ? 1.f : a.sm_scale, hf, glo, D, S3);
  }
}

// ------------------------------------------ dK/dV at head dims 64 and 256 --
// Each wave does all four products of its 32 keys (4 waves, 128 keys per
// workgroup), P and dS stay in registers, nothing goes through LDS between
// waves.  At D = 64 that fits 256 registers: two waves per SIMD and two
// workgroups per CU (the pair kernel's fp32 P exchange, 64 KiB whatever the
// head dim, holds it to one).  At D = 256 a 64-row tile is 32 KiB and the
// wave-pair kernel fits neither the LDS nor 256 registers per wave; there it
// runs one wave per SIMD (up to 512 registers) for the columns
// [D0, D0 + DH) of dK and dV: S^T and dP^T over the full head dim (B
// operands: this lane's K and V rows, 2 x 64 registers), then P, dS in
// registers and dV^T, dK^T for DH columns (A operands: dO^T and Q^T column
// blocks, read transposed).  Two launches (D0 = 0, 128) give the whole
// gradient, each recomputing S and dP.  Tiles are copied one step ahead into
// two slots (2 x 2 x 32 KiB).  With fp8 scores (Q8, at D = 64 and 256) S^T
// comes from an e4m3 Q8 tile and the lane's K8 row instead (QHALF below).
template <class E, int D, int NSP, int DH, int D0, bool Q8 = false>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void k_dkdv_wide(AttnArgs a, const uint32_t* __restrict__ codes,
                                                      const uint32_t* __restrict__ list,
                                                      const int32_t* __restrict__ count,
                                                      const uint32_t* __restrict__ order, int nT, int nKB) {
  constexpr bool SP = NSP >= 2, S3 = NSP == 3;
  using TL = Tile<D, 4>;
  // fp8 scores (Q8): S^T comes from the e4m3 Q8 tile and this lane's K8 row,
  // so the 16-bit Q tile feeds only dK^T += Q^T dS, i.e. only this launch's
  // columns [D0, D0 + DH): it is loaded DH wide (QHALF), which keeps the d = 256
  // launch's two slots of Q, Q8 and dO within the LDS
  constexpr bool QHALF = Q8 && DH < D;
  using TLQ = Tile<QHALF ? DH : D, 4>;    // 16-bit Q tiles
  using TQ8 = Tile<Q8 ? D / 2 : D, 4>;    // e4m3 Q tiles (D bytes a row), with Q8
  constexpr int DS = D / 16, NL = TL::LOADS_PER_WAVE, NLQ = TLQ::LOADS_PER_WAVE, NL8 = TQ8::LOADS_PER_WAVE;
  constexpr int HB = DH / 32, HB0 = D0 / 32;  // column blocks of this launch
  constexpr int NSL = 2;                      // slots per stream (copies one step ahead)
  __shared__ __attribute__((aligned(1024))) uint8_t s_q[NSL][TLQ::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_q8[Q8 ? NSL : 1][Q8 ? TQ8::BYTES : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t s_do[NSL][TL::BYTES];
  __shared__ __attribute__((aligned(256))) float s_lse[NSL][64];
  __shared__ __attribute__((aligned(256))) float s_delta[NSL][64];
  __shared__ __attribute__((aligned(256))) uint32_t s_qc[NSL][64];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, hf = lane >> 5,
            c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int h = work / (a.B * nKB);  // head-major, then the plan's longest-first dK/dV order
  const int item = int(order[work - h * (a.B * nKB)]);
  const int b = item / nKB, kblock = item - b * nKB, bh = b * H + h;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t qrb = uint32_t(a.q_strides[2]) * 2u, dorb = uint32_t(a.do_strides[2]) * 2u,
                 krb = uint32_t(a.k_strides[2]) * 2u, vrb = uint32_t(a.v_strides[2]) * 2u;
  const u32x4 rs_q = rsrc_words(qg, uint32_t(T) * qrb);
  const u32x4 rs_do = rsrc_words(dog, uint32_t(T) * dorb);
  const int64_t BHT = int64_t(a.B) * H * T;
  const u32x4 rs_lse = rsrc_words(a.delta + BHT + int64_t(bh) * T, uint32_t(T) * 4u);
  const u32x4 rs_dl = rsrc_words(a.delta + int64_t(bh) * T, uint32_t(T) * 4u);
  const u32x4 rs_codes = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);

  const int krow = kblock * 128 + wave * 32 + c;
  const bool kvalid = krow < T;
  // bytes of a row of the 16-bit inputs: 2 D, or fewer for head dims 16 and
  // 32 on the D = 64 kernel, whose other columns are read as zeros
  const uint32_t dbytes = uint32_t(a.D) * 2u;
  u32x4 bk[Q8 ? 1 : DS], bv[DS];  // this lane's K and V rows (B operands of S^T, dP^T)
  i32x8 bk8[Q8 ? D / 64 : 1];      // fp8: its K8 row instead, k-step st = bytes 64 st + 32 hf .. + 31
  {
    const auto rk = make_rsrc(kg, uint32_t(T) * krb), rv = make_rsrc(vg, uint32_t(T) * vrb);
#pragma unroll
    for (int st = 0; st < DS; ++st) {
      const uint32_t col = (16 * st + 8 * hf) * 2;
      if constexpr (!Q8) bk[st] = buf_load16(rk, col_masked(uint32_t(krow) * krb + col, col, dbytes));
      bv[st] = buf_load16(rv, col_masked(uint32_t(krow) * vrb + col, col, dbytes));
    }
    if constexpr (Q8) {
      const auto rs8 = make_rsrc(a.k8 + int64_t(bh) * T * D, uint32_t(T) * D);
#pragma unroll
      for (int st = 0; st < D / 64; ++st) {
        const u32x4 lo = buf_load16(rs8, uint32_t(krow) * D + 64 * st + 32 * hf);
        const u32x4 hi = buf_load16(rs8, uint32_t(krow) * D + 64 * st + 32 * hf + 16);
        bk8[st] = i32x8{int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]), int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
      }
    }
  }
  const int member = wave >> 1;
  uint32_t kcode = kvalid ? codes[int64_t(b) * T + krow] : 0u;

  const int lbase = b * nKB + kblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  uint32_t qoff[NLQ], dooff[NL], q8off[NL8];
  TLQ::load_offsets(wave, lane, qrb, qoff, QHALF ? uint32_t(DH) * 2u : dbytes);
  TL::load_offsets(wave, lane, dorb, dooff, dbytes);
  if constexpr (Q8) TQ8::load_offsets(wave, lane, uint32_t(D), q8off);
  const u32x4 rs_q8 = rsrc_words(Q8 ? a.q8 + int64_t(bh) * T * D : nullptr, Q8 ? uint32_t(T) * D : 0u);
  auto load_tile = [&](uint32_t en, int slot) {
    const uint32_t q0 = entry_tile(en) * 64u;
    // (QHALF: the tile's columns start at D0 of the row)
    TLQ::load_async(rs_q, q0 * qrb + (QHALF ? uint32_t(D0) * 2u : 0u), qoff, lds_addr(s_q[slot]), wave);
    TL::load_async(rs_do, q0 * dorb, dooff, lds_addr(s_do[slot]), wave);
    if constexpr (Q8) TQ8::load_async(rs_q8, q0 * uint32_t(D), q8off, lds_addr(s_q8[Q8 ? slot : 0]), wave);
    if (wave == 1)
      dma_b32(rs_lse, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_lse[slot][0])))));
    else if (wave == 2)
      dma_b32(rs_dl, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_delta[slot][0])))));
    else if (wave == 3)
      dma_b32(rs_codes, (q0 + lane) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_qc[slot][0])))));
  };

  const int srow = sigma(c);
  int raddr[DS];
#pragma unroll
  for (int st = 0; st < DS; ++st) raddr[st] = TL::at(srow, 2 * st + hf);
  int taddr_all[D / 32][2];
  tr_addrs<D>(lane, taddr_all);
  int taddr[HB][2];
#pragma unroll
  for (int db = 0; db < HB; ++db) {
    taddr[db][0] = taddr_all[HB0 + db][0];
    taddr[db][1] = taddr_all[HB0 + db][1];
  }
  // the transposed reads of the Q tile: as for dO, or the DH-wide tile's own blocks (QHALF)
  int taddr_q[HB][2];
  if constexpr (QHALF) {
    tr_addrs<DH>(lane, taddr_q);
  } else {
#pragma unroll
    for (int db = 0; db < HB; ++db) taddr_q[db][0] = taddr[db][0], taddr_q[db][1] = taddr[db][1];
  }

  // the fp8 product carries the dequantisation scales of Q and K
  const float sl2 = a.sm_scale * 1.4426950408889634f * (Q8 ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
  f32x16 acc_v[HB], acc_k[HB];  // dV^T, dK^T for this launch's columns
#pragma unroll
  for (int db = 0; db < HB; ++db) acc_v[db] = acc_k[db] = f32x16{};

  constexpr int PF = DKDV_PF;
  auto rows_times_b = [&](const uint8_t* ar_g, const u32x4 (&bop)[DS], f32x16 (&x)[2]) {
    lds_u8* ar = to_lds(ar_g);
    constexpr int NS = 2 * DS;
    auto read = [&](int i) { return ds_read16(ar + raddr[i >> 1] + (i & 1) * 32 * TL::ROWB); };
    u32x4 av[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      __builtin_amdgcn_sched_barrier(0x406);
      x[i & 1] = mfma32x32x16<E>(av[i % PF], bop[i >> 1], x[i & 1]);
      if (i + PF < NS) av[i % PF] = read(i + PF);
    }
    __builtin_amdgcn_sched_barrier(0x406);
  };
  // q_c: a std::integral_constant, true for the Q tile (TLQ's layout), false for dO
  auto accumulate = [&](const uint8_t* at_g, f32x16 (&acc)[HB], const u32x4 (&bop)[2][2],
                        const u32x4 (&bopl)[2][2], const u32x4 (&bopm)[2][2], auto q_c) {
    constexpr bool IS_Q = decltype(q_c)::value;
    constexpr int ROWB = IS_Q ? TLQ::ROWB : TL::ROWB;
    const int (&ta)[HB][2] = IS_Q ? taddr_q : taddr;
    lds_u8* at = to_lds(at_g);
    constexpr int NS = 4 * HB;
    auto read = [&](int i) {
      const int k4 = i / HB, db = i % HB, off = k4 * 16 * ROWB;
      const u32x2 lo = ds_read_tr16(at + ta[db][0] + off);
      const u32x2 hi = ds_read_tr16(at + ta[db][1] + off);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    u32x4 av[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) av[i] = read(i);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int k4 = i / HB, db = i % HB;
      __builtin_amdgcn_sched_barrier(0x406);
      acc[db] = mfma32x32x16<E>(av[i % PF], bop[k4 >> 1][k4 & 1], acc[db]);
      if constexpr (SP) acc[db] = mfma32x32x16<E>(av[i % PF], bopl[k4 >> 1][k4 & 1], acc[db]);
      if constexpr (S3) acc[db] = mfma32x32x16<E>(av[i % PF], bopm[k4 >> 1][k4 & 1], acc[db]);
      if (i + PF < NS) av[i % PF] = read(i + PF);
    }
    __builtin_amdgcn_sched_barrier(0x406);
  };
  auto splat_rows = [&](const float* v, f32x16 (&x)[2]) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ql = 32 * qb + 16 * t + 8 * hf;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(&v[ql]);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(&v[ql + 4]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[qb][8 * t + j] = l0[j];
          x[qb][8 * t + 4 + j] = l1[j];
        }
      }
  };

  if (n > 0) load_tile(ent[0], 0);
  wait_vmem();
#pragma unroll
  for (int st = 0; st < DS; ++st) {
    if constexpr (!Q8) settle(bk[st]);
    settle(bv[st]);
  }
  if constexpr (Q8) {
#pragma unroll
    for (int st = 0; st < D / 64; ++st) settle(bk8[st]);
  }
  settle(kcode);
  uint32_t en_cur = n > 0 ? ent[0] : 0u, en_next = n > 1 ? ent[1] : 0u;  // entries of tiles e, e + 1

  // One step per q-tile.  At D = 64 the loop is unrolled by two, so that the
  // slot of each step is a constant and every LDS address a fixed register
  // plus an immediate (19 fewer VALU instructions a step); at D = 256 the
  // unrolled loop spills, and the slot stays a loop variable.
  auto step = [&](const int e, auto slot_c) {
    const int slot = int(slot_c);  // == e & 1
    wait_vmem();   // tile e landed (the only copy in flight)
    barrier_lds(); // ... for every wave; every wave is done with tile e - 1
    uint32_t en = en_cur;
    asm volatile("" : "+s"(en));
    if (e + 1 < n) load_tile(en_next, slot ^ 1);
    en_cur = en_next;
    en_next = e + 2 < n ? ent[e + 2] : 0u;
    f32x16 x[2], y[2];  // S^T - LSE / c and dP^T - Delta
    splat_rows(s_lse[slot], x);
    splat_rows(s_delta[slot], y);
    if constexpr (Q8) {  // S^T = Q8 K8^T on the fp8 MFMA; A = Q8 rows, 32 bytes per lane and k-step
      const uint8_t* t8 = s_q8[Q8 ? slot : 0];
#pragma unroll
      for (int st = 0; st < D / 64; ++st) {
        const int a0 = TQ8::at(srow, 4 * st + 2 * hf), a1 = TQ8::at(srow, 4 * st + 2 * hf + 1);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const u32x4 lo = *reinterpret_cast<const u32x4*>(t8 + a0 + qb * 32 * TQ8::ROWB);
          const u32x4 hi = *reinterpret_cast<const u32x4*>(t8 + a1 + qb * 32 * TQ8::ROWB);
          const i32x8 av = {int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]), int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
          x[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bk8[st], x[qb], 0, 0, 0, 127, 0, 127);
        }
      }
    } else {
      rows_times_b(s_q[slot], bk, x);
    }
    rows_times_b(s_do[slot], bv, y);
    const uint32_t mcls = entry_class(en, member);
    if (mcls != TILE_FULL) {  // wave-uniform
      const uint64_t colbits = mcls == TILE_PARTIAL  // EMPTY: nothing allowed
                                   ? key_col_mask(kcode, krow, s_qc[slot][lane], int(entry_tile(en)) * 64)
                                   : 0u;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const uint32_t w = uint32_t(colbits >> (32 * qb)) >> (8 * hf);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[qb][r] = mask_bit(x[qb][r], w, 16 * (r >> 3) + (r & 7));
      }
    }
    u32x4 pb[2][2], pl[2][2], pm[2][2], sb[2][2], sl_[2][2], sm[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[8], ds[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          p[j] = fast_exp2(x[qb][8 * t + j] * sl2);
          ds[j] = p[j] * y[qb][8 * t + j];
        }
        pb[qb][t] = pack8<E>(p);
        sb[qb][t] = pack8<E>(ds);
        if constexpr (SP) {
          pl[qb][t] = pack8_residual<E>(p, pb[qb][t]);
          sl_[qb][t] = pack8_residual<E>(ds, sb[qb][t]);
        }
        if constexpr (S3) {
          pm[qb][t] = pack8_residual2<E>(p, pb[qb][t], pl[qb][t]);
          sm[qb][t] = pack8_residual2<E>(ds, sb[qb][t], sl_[qb][t]);
        }
      }
    accumulate(s_do[slot], acc_v, pb, pl, pm, std::false_type{});  // dV^T += dO^T P
    accumulate(s_q[slot], acc_k, sb, sl_, sm, std::true_type{});    // dK^T += Q^T dS
  };
  if constexpr (D <= 64) {
    for (int e = 0; e < n; e += 2) {
      step(e, std::integral_constant<int, 0>{});
      if (e + 1 < n) step(e + 1, std::integral_constant<int, 1>{});
    }
  } else {
    int slot = 0;
    for (int e = 0; e < n; ++e) {
      step(e, slot);
      slot ^= 1;
    }
  }

  if (kvalid) {
    uint16_t* gv = static_cast<uint16_t*>(a.dv) + b * a.dv_strides[0] + h * a.dv_strides[1] + krow * a.dv_strides[2];
    uint16_t* gk = static_cast<uint16_t*>(a.dk) + b * a.dk_strides[0] + h * a.dk_strides[1] + krow * a.dk_strides[2];
    const int64_t row = (int64_t(b) * a.H + h) * a.T + krow;
    auto lo_at = [&](void* base) {  // this launch's first column of the residual row
      void* r = lo_row(base, row, a.D, S3);
      return r == nullptr ? nullptr : static_cast<void*>(static_cast<uint8_t*>(r) + D0 * (S3 ? 4 : 2));
    };
    void* gv_lo = lo_at(a.dv_lo);
    void* gk_lo = lo_at(a.dk_lo);
    // (a.D < D only for the head dims 16 and 32 on the D = 64 launch, DH == D)
    store_rows_T<E, DH>(gv + D0, acc_v, 1.f, hf, gv_lo, DH == D ? a.D : DH, S3);
    if constexpr (DH == D) {  // all columns here: dK can be rotated back (dqk_signs)
      if (a.dqk_signs != nullptr) store_rows_T_unrot<E, D>(gk, acc_k, a.sm_scale, hf, a.dqk_signs);
      else store_rows_T<E, D>(gk, acc_k, a.sm_scale, hf, gk_lo, a.D, S3);
    } else {
      store_rows_T<E, DH>(gk + D0, acc_k, a.sm_scale, hf, gk_lo, DH, S3);  // (no dqk_signs at split widths)
    }
  }
}

// -------------------------------------------------------------- launchers --
template <class E, int D>
static void launch_delta_t(const AttnArgs& a, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  hipLaunchKernelGGL((k_delta<E, D>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
}
template <class E, int D, bool Q8, int NSP>
static void launch_dq_s(const AttnArgs& a, const uint8_t* plan, hipStream_t st, bool fuse_delta) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const unsigned grid = unsigned(a.B) * a.H * L.n_dq_blocks;
  auto* codes = reinterpret_cast<const uint32_t*>(plan + L.codes);
  auto* list = reinterpret_cast<const uint32_t*>(plan + L.dq_list);
  auto* cnt = reinterpret_cast<const int32_t*>(plan + L.dq_count);
  auto* order = reinterpret_cast<const uint32_t*>(plan + L.dq_order);
  if constexpr (D == 256) {  // two launches, the column halves of dQ; the first forms Delta
    hipLaunchKernelGGL((k_dq<E, D, Q8, NSP, 128, 0>), dim3(grid), dim3(256), 0, st, a, codes, list, cnt, order, L.nT,
                       L.n_dq_blocks, fuse_delta);
    hipLaunchKernelGGL((k_dq<E, D, Q8, NSP, 128, 128>), dim3(grid), dim3(256), 0, st, a, codes, list, cnt, order, L.nT,
                       L.n_dq_blocks, false);
  } else {
    hipLaunchKernelGGL((k_dq<E, D, Q8, NSP>), dim3(grid), dim3(256), 0, st, a, codes, list, cnt, order, L.nT,
                       L.n_dq_blocks, fuse_delta);
  }
}
template <class E, int D, bool Q8 = false>
static void launch_dq_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st, bool fuse_delta) {
  switch (parts_of(a.precision)) {
    case 1: launch_dq_s<E, D, Q8, 1>(a, plan, st, fuse_delta); break;
    case 2: launch_dq_s<E, D, Q8, 2>(a, plan, st, fuse_delta); break;
    default:
      if constexpr (!Q8) launch_dq_s<E, D, Q8, 3>(a, plan, st, fuse_delta);  // (refused with fp8 by the C ABI)
      break;
  }
}
template <class E, int D, bool Q8, int NSP>
static void launch_dkdv_s(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const unsigned grid = unsigned(a.B) * a.H * L.n_dkdv_blocks;
  if constexpr (D == 64) {  // one launch, all four products per wave (fp8 scores too)
    hipLaunchKernelGGL((k_dkdv_wide<E, D, NSP, 64, 0, Q8>), dim3(grid), dim3(256), 0, st, a,
                       reinterpret_cast<const uint32_t*>(plan + L.codes),
                       reinterpret_cast<const uint32_t*>(plan + L.dkdv_list),
                       reinterpret_cast<const int32_t*>(plan + L.dkdv_count),
                       reinterpret_cast<const uint32_t*>(plan + L.dkdv_order), L.nT, L.n_dkdv_blocks);
  } else if constexpr (D == 256) {  // two launches, the column halves of dK and dV (fp8 scores too)
    auto* codes = reinterpret_cast<const uint32_t*>(plan + L.codes);
    auto* list = reinterpret_cast<const uint32_t*>(plan + L.dkdv_list);
    auto* cnt = reinterpret_cast<const int32_t*>(plan + L.dkdv_count);
    auto* order = reinterpret_cast<const uint32_t*>(plan + L.dkdv_order);
    hipLaunchKernelGGL((k_dkdv_wide<E, D, NSP, 128, 0, Q8>), dim3(grid), dim3(256), 0, st, a, codes, list, cnt, order,
                       L.nT, L.n_dkdv_blocks);
    hipLaunchKernelGGL((k_dkdv_wide<E, D, NSP, 128, 128, Q8>), dim3(grid), dim3(256), 0, st, a, codes, list, cnt,
                       order, L.nT, L.n_dkdv_blocks);
  } else {
    hipLaunchKernelGGL((k_dkdv<E, D, Q8, NSP>), dim3(grid), dim3(512), 0, st, a,
                       reinterpret_cast<const uint32_t*>(plan + L.codes),
                       reinterpret_cast<const uint32_t*>(plan + L.dkdv_list),
                       reinterpret_cast<const int32_t*>(plan + L.dkdv_count),
                       reinterpret_cast<const uint32_t*>(plan + L.dkdv_order), L.nT, L.n_dkdv_blocks);
  }
}

template <class E, int D, bool Q8 = false>
static void launch_dkdv_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  switch (parts_of(a.precision)) {
    case 1: launch_dkdv_s<E, D, Q8, 1>(a, plan, st); break;
    case 2: launch_dkdv_s<E, D, Q8, 2>(a, plan, st); break;
    default:
      if constexpr (!Q8) launch_dkdv_s<E, D, Q8, 3>(a, plan, st);  // (refused with fp8 by the C ABI)
      break;
  }
}

// head dims 16 and 32 run on the D = 64 kernels (their rows read as zeros past a.D)
#define KD_DISPATCH(FN, ...)                                         \
  do {                                                               \
    if (a.dtype == KD_BF16) {                                        \
      if (a.D <= 64) FN<BF16, 64>(__VA_ARGS__);                      \
      else if (a.D == 128) FN<BF16, 128>(__VA_ARGS__);               \
      else FN<BF16, 256>(__VA_ARGS__);                               \
    } else {                                                         \
      if (a.D <= 64) FN<F16, 64>(__VA_ARGS__);                       \
      else if (a.D == 128) FN<F16, 128>(__VA_ARGS__);                \
      else FN<F16, 256>(__VA_ARGS__);                                \
    }                                                                \
  } while (0)

template <class E>
static void launch_delta_e(const AttnArgs& a, hipStream_t st) {
  switch (a.D) {  // k_delta reads whole rows of a.D elements
    case 16: launch_delta_t<E, 16>(a, st); break;
    case 32: launch_delta_t<E, 32>(a, st); break;
    case 64: launch_delta_t<E, 64>(a, st); break;
    case 128: launch_delta_t<E, 128>(a, st); break;
    default: launch_delta_t<E, 256>(a, st); break;
  }
}

int launch_delta(const AttnArgs& a, hipStream_t st) {
  if (use_simt(a)) return launch_simt_kernel(1, a, nullptr, st);
  if (a.dtype == KD_BF16) launch_delta_e<BF16>(a, st);
  else launch_delta_e<F16>(a, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}
int launch_dq(const AttnArgs& a, const uint8_t* plan, hipStream_t st, bool fuse_delta) {
  if (use_simt(a)) {
    const int r = fuse_delta ? launch_simt_kernel(1, a, plan, st) : KD_OK;
    return r ? r : launch_simt_kernel(2, a, plan, st);
  }
  if (a.q8 != nullptr) {  // fp8 QK^T: bf16 at head dim 64, 128 or 256 (checked by the C ABI)
    if (a.D == 64) launch_dq_t<BF16, 64, true>(a, plan, st, fuse_delta);
    else if (a.D == 128) launch_dq_t<BF16, 128, true>(a, plan, st, fuse_delta);
    else launch_dq_t<BF16, 256, true>(a, plan, st, fuse_delta);
  }
  else KD_DISPATCH(launch_dq_t, a, plan, st, fuse_delta);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}
int launch_dkdv(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (use_simt(a)) return launch_simt_kernel(3, a, plan, st);
  if (a.q8 != nullptr) {  // fp8 QK^T: bf16 at head dim 64, 128 or 256 (checked by the C ABI)
    if (a.D == 64) launch_dkdv_t<BF16, 64, true>(a, plan, st);
    else if (a.D == 128) launch_dkdv_t<BF16, 128, true>(a, plan, st);
    else launch_dkdv_t<BF16, 256, true>(a, plan, st);
  }
  else KD_DISPATCH(launch_dkdv_t, a, plan, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
