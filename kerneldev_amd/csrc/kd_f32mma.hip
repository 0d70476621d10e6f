// Attention for fp32 inputs on the fp32 matrix cores (v_mfma_f32_32x32x2_f32):
// the reference's fp32 dots (original_kernel.py:452, :569, :1239, :1331-1333,
// :1425, :1517-1523) with fp32 operands and fp32 accumulation, at head dim 32
// (and 16, zero-padded to 32 by the Python layer; head dims 64, 128 and 256
// run on the 16 x 16 form of kd_f32w.hip).  The kernels are templates over the
// head dim and were built for 64 and 128 too.  Same algebra, plan, lists and masks as the 16-bit kernels:
//   forward   O = softmax2(S c) V, LSE2 = m + log2 l      (:279-626)
//   dQ        P = exp2(S c - LSE), dS = P (dP - Delta), dQ = sm_scale dS K  (:1173-1336)
//   dK / dV   dV = P^T dO, dK = sm_scale dS^T Q            (:1339-1525)
// with c = sm_scale log2(e) folded into the register-resident Q (forward,
// dQ) or K (dK/dV) as the vector-ALU kernels do.  Delta comes from
// k_delta_simt (kd_simt.hip).
//
// The fp32 MFMA.  D += A B with A 32 x 2 and B 2 x 32: lane (c = lane % 32,
// h = lane / 32) supplies A[c][h] and B[h][c], and register r of the 32 x 32
// result holds row row_of(r, h) = 8 (r / 4) + 4 h + r % 4, column c.  One
// instruction is 4096 FLOP, so the product over a head dim D takes D / 2
// k-steps; k-step 4u + t contracts column 8u + 4h + t on lane half h, so a
// lane reads its A row's four columns of four consecutive k-steps with one
// 16-byte LDS read, and the register-resident operand (the lane's own Q, K,
// V or dO row) is held in that order.  Every product keeps the tile's tokens
// on the rows of the result, the wave's own 32 tokens on its columns:
//   forward, dQ:  S^T[key][query] = K Q^T, dP^T = V dO^T: each lane owns one
//                 query (its column), so the softmax statistics, LSE and
//                 Delta are per-lane scalars (plus one half-wave swap);
//                 O^T / dQ^T [d][query] += V^T / K^T [d][key] P^T / dS^T,
//                 whose B operand is register r of the S^T accumulators for
//                 k-step 16 kb + r (keys 32 kb + row_of(r, h)), and whose A
//                 operand is one float of the V / K tile per k-step.
//   dK/dV:        S[query][key] = Q K^T, dP = dO V^T, each lane owning one
//                 key; dV^T / dK^T [d][key] += dO^T / Q^T [d][query] P / dS.
// Workgroup: 4 waves x 32 tokens = one 128-token block of the plan's lists;
// member tile = wave / 2; blocks are taken head-major (each XCD one range of
// heads, xcd_remap) and, for the forward and dQ, in the plan's longest-first
// order.  Streamed 64-token tiles (fp32 rows, 16-byte chunks
// XOR-swizzled per row as in kd_tile.h) are copied global -> LDS with
// buffer_load ... lds one step ahead into two slots; an EMPTY member tile
// skips its wave's products, a PARTIAL one evaluates allow() per score from
// the token codes.
#include "kd_tile.h"

namespace kd {
namespace {

KD_DEV f32x16 mma_f32(float a, float b, const f32x16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
}
KD_DEV int row_of(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// 64 rows x D floats: the 16-bit tile machinery with rows of 2 D halves
template <int D>
struct F32Tile {
  using TL = Tile<2 * D, 4>;
  static constexpr int BYTES = TL::BYTES;
  // byte offset of float (r, col)
  KD_DEV static int at(int r, int col) { return TL::at(r, col >> 2) + ((col & 3) << 2); }
  // this wave's share of the copy of rows r0 .. r0 + 63 of a slice with
  // row_bytes bytes a row; arow / c16 from lane_row / lane_chunk16
  KD_DEV static void copy(const u32x4& rs, uint32_t r0, uint32_t row_bytes, uint32_t arow, uint32_t c16,
                          const uint8_t* lds_tile, int wave) {
    TL::load_async_rows(rs, r0 * row_bytes, arow, c16, row_bytes, lds_addr(lds_tile), wave);
  }
};

// this lane's row x[row][.] in k-step order: out[4u + t] = x[row][8u + 4h + t] * scale
template <int D>
KD_DEV void load_row(const float* base, int64_t row_stride, int row, bool valid, int h, float scale, float (&out)[D / 2]) {
  const float* p = base + int64_t(valid ? row : 0) * row_stride + 4 * h;  // row 0 stands in past T
  const float sc = valid ? scale : 0.f;
#pragma unroll
  for (int u = 0; u < D / 8; ++u) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(p + 8 * u);
#pragma unroll
    for (int t = 0; t < 4; ++t) out[4 * u + t] = x[t] * sc;
  }
}

// S^T (or S) of one 32-row block of an LDS tile against the lane's register row:
// acc[r] = sum_d tile[32 kb + row_of(r, h)][d] * reg-row[d].  Each 16-byte read
// is issued one group of four MFMAs ahead of its use; the fences keep the
// compiler from hoisting every read of the product (and holding its values)
template <int D>
KD_DEV f32x16 score_block(const uint8_t* tile, int kb, int c, int h, const float (&reg)[D / 2]) {
  f32x16 acc = {};
  using TL = typename F32Tile<D>::TL;
  const uint8_t* row = tile + (32 * kb + c) * TL::ROWB;  // chunk q of the row is at (q ^ swz) * 16
  const int sw = TL::swz(32 * kb + c);
  f32x4 a = *reinterpret_cast<const f32x4*>(row + ((h ^ sw) << 4));
#pragma unroll
  for (int u = 0; u < D / 8; ++u) {
    f32x4 nx = a;
    if (u + 1 < D / 8) nx = *reinterpret_cast<const f32x4*>(row + (((2 * (u + 1) + h) ^ sw) << 4));
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = mma_f32(a[t], reg[4 * u + t], acc);
    __builtin_amdgcn_sched_barrier(0);
    a = nx;
  }
  return acc;
}

// acc[db] (the [d][token] product's 32-row block db) += tile^T B over the
// tile's rows 32 kb .. 32 kb + 31, B = the score-shaped registers s (row
// 32 kb + row_of(r, h) in register r), with the one-float A reads issued a
// group of four k-steps ahead
template <int D>
KD_DEV void accumulate_blk(const uint8_t* tile, int kb, int c, int h, const f32x16& s, f32x16 (&acc)[D / 32]) {
  constexpr int NS = 16 * (D / 32);  // k-steps over all blocks: i = 16 db + r
  auto rd = [&](int i) {
    return *reinterpret_cast<const float*>(tile + F32Tile<D>::at(32 * kb + row_of(i & 15, h), 32 * (i >> 4) + c));
  };
  float a[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) a[t] = rd(t);
#pragma unroll
  for (int i0 = 0; i0 < NS; i0 += 4) {
    float nx[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) nx[t] = i0 + 4 < NS ? rd(i0 + 4 + t) : a[t];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = i0 + t;
      acc[i >> 4] = mma_f32(a[t], s[i & 15], acc[i >> 4]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) a[t] = nx[t];
  }
}

// store the [d][token] accumulators of this lane's token (column c) to row
// `row` of out, times scale: register 4 g + i of block db is column 32 db + 8 g + 4 h + i
template <int D>
KD_DEV void store_t(float* out, const f32x16 (&acc)[D / 32], int h, float scale) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 x = {acc[db][4 * g] * scale, acc[db][4 * g + 1] * scale, acc[db][4 * g + 2] * scale,
                       acc[db][4 * g + 3] * scale};
      *reinterpret_cast<f32x4*>(out + 32 * db + 8 * g + 4 * h) = x;
    }
}

// ------------------------------------------------------------------ forward
template <int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void k_fwd_f32m(AttnArgs a, const uint32_t* __restrict__ codes,
                                                                   const uint32_t* __restrict__ list,
                                                                   const int32_t* __restrict__ count, int nT, int nblk,
    const uint32_t* __restrict__ order) {
  using FT = F32Tile<D>;
  constexpr int DB = D / 32;
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][FT::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][FT::BYTES];
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), member = wave >> 1;
  // head-major, then the plan's longest-first order of (batch row, block)
  const int work = xcd_remap(blockIdx.x, gridDim.x), T = a.T;
  const int hh = work / (a.B * nblk), item = int(order[work - hh * (a.B * nblk)]);
  const int b = item / nblk, blk = item - b * nblk, bh = b * a.H + hh;
  const int q = blk * 128 + wave * 32 + c;  // this lane's query
  const bool qvalid = q < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + b * a.q_strides[0] + hh * a.q_strides[1];
  const float* kg = static_cast<const float*>(a.k) + b * a.k_strides[0] + hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + b * a.v_strides[0] + hh * a.v_strides[1];
  const uint32_t krb = uint32_t(a.k_strides[2]) * 4u, vrb = uint32_t(a.v_strides[2]) * 4u;
  const u32x4 rs_k = rsrc_words(kg, uint32_t(T) * krb), rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  const uint32_t c16 = FT::TL::lane_chunk16(wave, lane), lrow = FT::TL::lane_row(wave, lane);
  uint32_t qcode = qvalid ? codes[int64_t(b) * T + q] : 0u;

  float qr[D / 2];
  load_row<D>(qg, a.q_strides[2], q, qvalid, h, cs, qr);

  const int lb = b * nblk + blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  auto copy = [&](uint32_t en, int slot) {
    const uint32_t r0 = entry_tile(en) * 64u;
    FT::copy(rs_k, r0, krb, lrow * krb, c16, s_k[slot], wave);
    FT::copy(rs_v, r0, vrb, lrow * vrb, c16, s_v[slot], wave);
    if (wave == 0) dma_b32(rs_c, (r0 + uint32_t(lane)) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_kc[slot])))));
  };
  if (n > 0) copy(ent[0], 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < D / 2; ++j) settle(qr[j]);
  settle(qcode);

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  float m = -__builtin_inff(), l = 0.f;
  for (int e = 0; e < n; ++e) {
    const int slot = e & 1;
    wait_vmem();
    const uint32_t en = ent[e];
    const uint32_t en_next = e + 1 < n ? ent[e + 1] : 0u;
    barrier_raw();  // tile e landed for every wave; every wave is done with tile e - 1
    if (e + 1 < n) copy(en_next, slot ^ 1);
    const uint32_t cls = entry_class(en, member);
    if (cls == TILE_EMPTY) continue;  // wave-uniform: nothing of this tile is allowed for these rows
    const uint8_t* kt = s_k[slot];
    const uint8_t* vt = s_v[slot];
    f32x16 s[2];
    s[0] = score_block<D>(kt, 0, c, h, qr);
    s[1] = score_block<D>(kt, 1, c, h, qr);
    if (cls == TILE_PARTIAL) {
      const int k0 = int(entry_tile(en)) * 64;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 kc = *reinterpret_cast<const u32x4*>(&s_kc[slot][32 * kb + 8 * g + 4 * h]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            s[kb][4 * g + i] = allow(qcode, kc[i], q, k0 + 32 * kb + 8 * g + 4 * h + i) ? s[kb][4 * g + i]
                                                                                       : -__builtin_inff();
        }
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    const float m_new = fmaxf(m, xhalf_max(mx));
    const float mu = m_new == -__builtin_inff() ? 0.f : m_new;  // rows with nothing allowed yet keep P = 0
    const float alpha = fast_exp2(m - mu);                       // 0 while m is -inf
    m = m_new;
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[kb][r] = fast_exp2(s[kb][r] - mu);
        ls += s[kb][r];
      }
    l = l * alpha + xhalf_sum(ls);
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;
    accumulate_blk<D>(vt, 0, c, h, s[0], o);
    accumulate_blk<D>(vt, 1, c, h, s[1], o);
  }
  if (!qvalid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  store_t<D>(static_cast<float*>(a.o) + b * a.o_strides[0] + hh * a.o_strides[1] + int64_t(q) * a.o_strides[2], o, h,
             inv);
  if (h == 0 && a.lse != nullptr) a.lse[int64_t(bh) * T + q] = l > 0.f ? m + fast_log2(l) : -__builtin_inff();
}

// ----------------------------------------------------------------------- dQ
template <int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void k_dq_f32m(AttnArgs a, const uint32_t* __restrict__ codes,
                                                                  const uint32_t* __restrict__ list,
                                                                  const int32_t* __restrict__ count, int nT, int nblk,
    const uint32_t* __restrict__ order) {
  using FT = F32Tile<D>;
  constexpr int DB = D / 32;
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][FT::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][FT::BYTES];
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), member = wave >> 1;
  // head-major, then the plan's longest-first order of (batch row, block)
  const int work = xcd_remap(blockIdx.x, gridDim.x), T = a.T;
  const int hh = work / (a.B * nblk), item = int(order[work - hh * (a.B * nblk)]);
  const int b = item / nblk, blk = item - b * nblk, bh = b * a.H + hh;
  const int q = blk * 128 + wave * 32 + c;
  const bool qvalid = q < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + b * a.q_strides[0] + hh * a.q_strides[1];
  const float* dog = static_cast<const float*>(a.dout) + b * a.do_strides[0] + hh * a.do_strides[1];
  const float* kg = static_cast<const float*>(a.k) + b * a.k_strides[0] + hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + b * a.v_strides[0] + hh * a.v_strides[1];
  const uint32_t krb = uint32_t(a.k_strides[2]) * 4u, vrb = uint32_t(a.v_strides[2]) * 4u;
  const u32x4 rs_k = rsrc_words(kg, uint32_t(T) * krb), rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  const uint32_t c16 = FT::TL::lane_chunk16(wave, lane), lrow = FT::TL::lane_row(wave, lane);
  uint32_t qcode = qvalid ? codes[int64_t(b) * T + q] : 0u;
  // P = exp2(S c - LSE); a fully masked row (LSE = -inf) gets P = 0
  const float l0 = qvalid ? a.lse[int64_t(bh) * T + q] : -__builtin_inff();
  float lse = l0 == -__builtin_inff() ? __builtin_inff() : l0;
  float ndelta = qvalid ? a.delta[int64_t(bh) * T + q] : 0.f;  // the workspace holds -Delta

  float qr[D / 2], dr[D / 2];
  load_row<D>(qg, a.q_strides[2], q, qvalid, h, cs, qr);
  load_row<D>(dog, a.do_strides[2], q, qvalid, h, 1.f, dr);

  const int lb = b * nblk + blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  auto copy = [&](uint32_t en, int slot) {
    const uint32_t r0 = entry_tile(en) * 64u;
    FT::copy(rs_k, r0, krb, lrow * krb, c16, s_k[slot], wave);
    FT::copy(rs_v, r0, vrb, lrow * vrb, c16, s_v[slot], wave);
    if (wave == 0) dma_b32(rs_c, (r0 + uint32_t(lane)) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_kc[slot])))));
  };
  if (n > 0) copy(ent[0], 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < D / 2; ++j) {
    settle(qr[j]);
    settle(dr[j]);
  }
  settle(qcode);
  settle(lse);
  settle(ndelta);

  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = f32x16{};
  for (int e = 0; e < n; ++e) {
    const int slot = e & 1;
    wait_vmem();
    const uint32_t en = ent[e];
    const uint32_t en_next = e + 1 < n ? ent[e + 1] : 0u;
    barrier_raw();
    if (e + 1 < n) copy(en_next, slot ^ 1);
    const uint32_t cls = entry_class(en, member);
    if (cls == TILE_EMPTY) continue;
    const uint8_t* kt = s_k[slot];
    const uint8_t* vt = s_v[slot];
    f32x16 s[2], dp[2];
    s[0] = score_block<D>(kt, 0, c, h, qr);
    s[1] = score_block<D>(kt, 1, c, h, qr);
    dp[0] = score_block<D>(vt, 0, c, h, dr);
    dp[1] = score_block<D>(vt, 1, c, h, dr);
    if (cls == TILE_PARTIAL) {
      const int k0 = int(entry_tile(en)) * 64;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 kc = *reinterpret_cast<const u32x4*>(&s_kc[slot][32 * kb + 8 * g + 4 * h]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            s[kb][4 * g + i] = allow(qcode, kc[i], q, k0 + 32 * kb + 8 * g + 4 * h + i) ? s[kb][4 * g + i]
                                                                                       : -__builtin_inff();
        }
    }
    // dS^T = P^T (dP^T - Delta), in place of S^T
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = fast_exp2(s[kb][r] - lse) * (dp[kb][r] + ndelta);
    accumulate_blk<D>(kt, 0, c, h, s[0], dq);
    accumulate_blk<D>(kt, 1, c, h, s[1], dq);
  }
  if (!qvalid) return;
  store_t<D>(static_cast<float*>(a.dq) + b * a.dq_strides[0] + hh * a.dq_strides[1] + int64_t(q) * a.dq_strides[2], dq,
             h, a.sm_scale);
}

// -------------------------------------------------------------------- dK/dV
template <int D>
__global__ __launch_bounds__(256, D <= 32 ? 2 : 1) void k_dkdv_f32m(AttnArgs a, const uint32_t* __restrict__ codes,
                                                                    const uint32_t* __restrict__ list,
                                                                    const int32_t* __restrict__ count, int nT,
                                                                    int nblk, const uint32_t* __restrict__ order) {
  using FT = F32Tile<D>;
  constexpr int DB = D / 32;
  __shared__ __attribute__((aligned(1024))) uint8_t s_q[2][FT::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_do[2][FT::BYTES];
  __shared__ __attribute__((aligned(256))) float s_lse[2][64];
  __shared__ __attribute__((aligned(256))) float s_dl[2][64];
  __shared__ __attribute__((aligned(256))) uint32_t s_qc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), member = wave >> 1;
  // head-major, then the plan's longest-first dK/dV order
  const int work = xcd_remap(blockIdx.x, gridDim.x), T = a.T;
  const int hh = work / (a.B * nblk), item = int(order[work - hh * (a.B * nblk)]);
  const int b = item / nblk, blk = item - b * nblk, bh = b * a.H + hh;
  const int k = blk * 128 + wave * 32 + c;  // this lane's key
  const bool kvalid = k < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + b * a.q_strides[0] + hh * a.q_strides[1];
  const float* dog = static_cast<const float*>(a.dout) + b * a.do_strides[0] + hh * a.do_strides[1];
  const float* kg = static_cast<const float*>(a.k) + b * a.k_strides[0] + hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + b * a.v_strides[0] + hh * a.v_strides[1];
  const uint32_t qrb = uint32_t(a.q_strides[2]) * 4u, dorb = uint32_t(a.do_strides[2]) * 4u;
  const u32x4 rs_q = rsrc_words(qg, uint32_t(T) * qrb), rs_do = rsrc_words(dog, uint32_t(T) * dorb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  const u32x4 rs_l = rsrc_words(a.lse + int64_t(bh) * T, uint32_t(T) * 4u);
  const u32x4 rs_d = rsrc_words(a.delta + int64_t(bh) * T, uint32_t(T) * 4u);  // -Delta
  const uint32_t c16 = FT::TL::lane_chunk16(wave, lane), lrow = FT::TL::lane_row(wave, lane);
  uint32_t kcode = kvalid ? codes[int64_t(b) * T + k] : 0u;

  float kr[D / 2], vr[D / 2];
  load_row<D>(kg, a.k_strides[2], k, kvalid, h, cs, kr);
  load_row<D>(vg, a.v_strides[2], k, kvalid, h, 1.f, vr);

  const int lb = b * nblk + blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  auto copy = [&](uint32_t en, int slot) {
    const uint32_t r0 = entry_tile(en) * 64u;
    FT::copy(rs_q, r0, qrb, lrow * qrb, c16, s_q[slot], wave);
    FT::copy(rs_do, r0, dorb, lrow * dorb, c16, s_do[slot], wave);
    const uint32_t off = (r0 + uint32_t(lane)) * 4u;
    if (wave == 0) dma_b32(rs_c, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_qc[slot])))));
    if (wave == 1) dma_b32(rs_l, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_lse[slot])))));
    if (wave == 2) dma_b32(rs_d, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_dl[slot])))));
  };
  if (n > 0) copy(ent[0], 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < D / 2; ++j) {
    settle(kr[j]);
    settle(vr[j]);
  }
  settle(kcode);

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dk[db] = dv[db] = f32x16{};
  for (int e = 0; e < n; ++e) {
    const int slot = e & 1;
    wait_vmem();
    const uint32_t en = ent[e];
    const uint32_t en_next = e + 1 < n ? ent[e + 1] : 0u;
    barrier_raw();
    if (e + 1 < n) copy(en_next, slot ^ 1);
    const uint32_t cls = entry_class(en, member);
    if (cls == TILE_EMPTY) continue;
    const uint8_t* qt = s_q[slot];
    const uint8_t* dt = s_do[slot];
    const int q0 = int(entry_tile(en)) * 64;
    const bool full = cls == TILE_FULL;
    for (int qb = 0; qb < 2; ++qb) {  // one 32-query block at a time (registers)
      f32x16 s = score_block<D>(qt, qb, c, h, kr);
      f32x16 dp = score_block<D>(dt, qb, c, h, vr);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = 32 * qb + 8 * g + 4 * h;  // rows row .. row + 3 are registers 4 g .. 4 g + 3
        const f32x4 lv = *reinterpret_cast<const f32x4*>(&s_lse[slot][row]);
        const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&s_dl[slot][row]);
        // (branch-free per element: bitwise logic and selects; the mask rule
        // only in PARTIAL tiles, a wave-uniform branch)
        bool ok[4];
        if (full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) ok[i] = lv[i] != -__builtin_inff();
        } else {
          const u32x4 qc = *reinterpret_cast<const u32x4*>(&s_qc[slot][row]);
#pragma unroll
          for (int i = 0; i < 4; ++i) ok[i] = (lv[i] != -__builtin_inff()) & allow(qc[i], kcode, q0 + row + i, k);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ex = fast_exp2(s[4 * g + i] - lv[i]);
          const float p = ok[i] ? ex : 0.f;
          s[4 * g + i] = p;
          dp[4 * g + i] = p * (dp[4 * g + i] + dv4[i]);  // dS
        }
      }
      accumulate_blk<D>(dt, qb, c, h, s, dv);
      accumulate_blk<D>(qt, qb, c, h, dp, dk);
    }
  }
  if (!kvalid) return;
  store_t<D>(static_cast<float*>(a.dk) + b * a.dk_strides[0] + hh * a.dk_strides[1] + int64_t(k) * a.dk_strides[2], dk,
             h, a.sm_scale);
  store_t<D>(static_cast<float*>(a.dv) + b * a.dv_strides[0] + hh * a.dv_strides[1] + int64_t(k) * a.dv_strides[2], dv,
             h, 1.f);
}

template <int D>
void launch_f32m_d(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const uint32_t* codes = reinterpret_cast<const uint32_t*>(plan + L.codes);
  auto lst = [&](size_t off) { return reinterpret_cast<const uint32_t*>(plan + off); };
  auto cnt = [&](size_t off) { return reinterpret_cast<const int32_t*>(plan + off); };
  const unsigned bh = unsigned(a.B) * unsigned(a.H);
  if (which == 0)
    hipLaunchKernelGGL((k_fwd_f32m<D>), dim3(bh * unsigned(L.n_fwd_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.fwd_list), cnt(L.fwd_count), L.nT, L.n_fwd_blocks, lst(L.fwd_order));
  else if (which == 2)
    hipLaunchKernelGGL((k_dq_f32m<D>), dim3(bh * unsigned(L.n_dq_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.dq_list), cnt(L.dq_count), L.nT, L.n_dq_blocks, lst(L.dq_order));
  else
    hipLaunchKernelGGL((k_dkdv_f32m<D>), dim3(bh * unsigned(L.n_dkdv_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.dkdv_list), cnt(L.dkdv_count), L.nT, L.n_dkdv_blocks, lst(L.dkdv_order));
}

}  // namespace

bool use_f32mma(const AttnArgs& a) {
  return a.dtype == KD_F32 && (a.D == 32 || a.D == 64 || a.D == 128 || a.D == 256);
}

// Head dim 32 here; 64, 128 and 256 on the 16 x 16 form (kd_f32w.hip), which
// runs them 5-16% faster (d = 64, 128) and fits 256 at all.
int launch_f32mma(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (a.D != 32) return launch_f32w(which, a, plan, st);
  launch_f32m_d<32>(which, a, plan, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
