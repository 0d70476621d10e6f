// Backward of the hierarchical-mask flash attention on gfx950 MFMA.
//
// Algebra of original_kernel.py:1239-1335 (dQ) and :1425-1524 (dK/dV), with
// P recomputed from the saved base-2 LSE, Delta = rowsum(O * dO) (:695) and
// the tile map driving both loops.  Unlike the reference with causal=True
// (:1199-1207, :1366-1375) the loops visit EVERY non-empty tile, so the
// gradient is the true gradient of the forward's mask.
//
// dQ kernel: 4 waves x 32 query rows per workgroup, 64 keys per step:
//   S^T  = K Q^T,  dP^T = V dO^T          (A = K, V rows from LDS; B = Q, dO regs)
//   dS^T = P^T * (dP^T - Delta)            (per-lane Delta, LSE)
//   dQ^T += K^T dS^T                       (A = K^T from LDS; B = dS regs)
// dK/dV kernel: 4 waves x 32 keys per workgroup, 64 queries per step:
//   S = Q K^T,  dP = dO V^T                (A = Q, dO rows from LDS; B = K, V regs)
//   dV^T += dO^T P,  dK^T += Q^T dS        (A = dO^T, Q^T from LDS; B = P, dS regs)
// Both keep the accumulated gradient transposed in registers so the MFMA
// output of one product is the register-resident B operand of the next.
#include "kd_internal.h"

namespace kd {

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
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      sum += to_f32<E>(uint16_t(ov[w] & 0xFFFFu)) * to_f32<E>(uint16_t(dv[w] & 0xFFFFu));
      sum += to_f32<E>(uint16_t(ov[w] >> 16)) * to_f32<E>(uint16_t(dv[w] >> 16));
    }
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (row < nrows && seg == 0) a.delta[row] = sum;
}

// ------------------------------------------------------------ shared cfg ----
template <int D>
struct BwdCfg {
  static constexpr int BN = 64;              // keys (dQ) or queries (dK/dV) per step
  static constexpr int RST = D + 8;          // row-major tile stride (elements)
  static constexpr int TST = BN + 8;         // transposed tile stride (elements)
  static constexpr int DS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int BLK = (BN / 4) * (D / 8);   // 4-row x 8-col blocks per tile
  static constexpr int R_ELEMS = BN * RST;
  static constexpr int T_ELEMS = D * TST;
};

// Load one 4-row x 8-col block of a [BN, D] tile (rows r0.., 16-byte loads).
template <int D>
KD_DEV void load_block(const uint16_t* base, int64_t rstride, int row0, int T, int blk, u32x4 (&r)[4]) {
  const int rg = blk / (D / 8), dc = blk % (D / 8);
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int row = row0 + 4 * rg + x;
    r[x] = row < T ? *reinterpret_cast<const u32x4*>(base + row * rstride + dc * 8) : u32x4{0, 0, 0, 0};
  }
}
// Store it row-major ([BN][RST]) and transposed ([D][TST]).
template <int D>
KD_DEV void store_block(uint16_t* rm, uint16_t* tr, int blk, const u32x4 (&r)[4]) {
  using C = BwdCfg<D>;
  const int rg = blk / (D / 8), dc = blk % (D / 8);
  if (rm != nullptr) {
#pragma unroll
    for (int x = 0; x < 4; ++x) *reinterpret_cast<u32x4*>(&rm[(4 * rg + x) * C::RST + dc * 8]) = r[x];
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    u32x2 lo = {pack_lo(r[0][w], r[1][w]), pack_lo(r[2][w], r[3][w])};
    u32x2 hi = {pack_hi(r[0][w], r[1][w]), pack_hi(r[2][w], r[3][w])};
    *reinterpret_cast<u32x2*>(&tr[(8 * dc + 2 * w) * C::TST + 4 * rg]) = lo;
    *reinterpret_cast<u32x2*>(&tr[(8 * dc + 2 * w + 1) * C::TST + 4 * rg]) = hi;
  }
}

template <class E, int D>
KD_DEV void store_rows_T(uint16_t* g, const f32x16 (&acc)[D / 32], float scale, int hf) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      const int d0 = 32 * db + 8 * gg + 4 * hf;
      u32x2 w = {pack2<E>(acc[db][4 * gg] * scale, acc[db][4 * gg + 1] * scale),
                 pack2<E>(acc[db][4 * gg + 2] * scale, acc[db][4 * gg + 3] * scale)};
      *reinterpret_cast<u32x2*>(g + d0) = w;
    }
  }
}

// ------------------------------------------------------------------- dQ ----
template <class E, int D>
__global__ __launch_bounds__(256) void k_dq(AttnArgs a, const uint32_t* __restrict__ codes,
                                            const uint32_t* __restrict__ list,
                                            const int32_t* __restrict__ count, int nT, int nQB) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][C::R_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[2][C::R_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_kt[2][C::T_ELEMS];
  __shared__ __attribute__((aligned(16))) uint32_t s_code[2][C::BN];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / nQB;
  const int qblock = nQB - 1 - (work % nQB);
  const int b = bh / H, h = bh % H;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t* codes_b = codes + int64_t(b) * T;

  const int qrow = qblock * 128 + wave * 32 + c;
  const bool qvalid = qrow < T;
  u32x4 qf[C::DS], dof[C::DS];
#pragma unroll
  for (int st = 0; st < C::DS; ++st) {
    qf[st] = qvalid ? *reinterpret_cast<const u32x4*>(qg + qrow * a.q_strides[2] + 16 * st + 8 * hf)
                    : u32x4{0, 0, 0, 0};
    dof[st] = qvalid ? *reinterpret_cast<const u32x4*>(dog + qrow * a.do_strides[2] + 16 * st + 8 * hf)
                     : u32x4{0, 0, 0, 0};
  }
  const float INF = __builtin_inff();
  float lse = qvalid ? a.lse[int64_t(bh) * T + qrow] : -INF;
  lse = (lse == -INF) ? INF : lse;  // fully masked row: every p becomes 0
  const float delta = qvalid ? a.delta[int64_t(bh) * T + qrow] : 0.f;
  const uint32_t qcode = qvalid ? codes_b[qrow] : 0u;

  const int lbase = b * nQB + qblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  // K via 4x8 blocks (row-major + transposed), V via the same blocks (row-major)
  u32x4 rk[4], rv[4];
  uint32_t rcode = 0;
  auto load_tile = [&](int kt) {
    const int k0 = kt * C::BN;
    if (tid < C::BLK) {
      load_block<D>(kg, a.k_strides[2], k0, T, tid, rk);
      load_block<D>(vg, a.v_strides[2], k0, T, tid, rv);
    }
    if (tid < C::BN) rcode = (k0 + tid < T) ? codes_b[k0 + tid] : 0u;
  };
  auto store_tile = [&](int buf) {
    if (tid < C::BLK) {
      store_block<D>(s_k[buf], s_kt[buf], tid, rk);
      const int rg = tid / (D / 8), dc = tid % (D / 8);
#pragma unroll
      for (int x = 0; x < 4; ++x) *reinterpret_cast<u32x4*>(&s_v[buf][(4 * rg + x) * C::RST + dc * 8]) = rv[x];
    }
    if (tid < C::BN) s_code[buf][tid] = rcode;
  };

  const float sl2 = a.sm_scale * 1.4426950408889634f;
  const float NEG_INF = -INF;
  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};
  const int srow = sigma(c);

  if (n > 0) {
    load_tile(int(ent[0] >> 1));
    store_tile(0);
  }
  __syncthreads();

  for (int e = 0; e < n; ++e) {
    const int buf = e & 1;
    const uint32_t cur = ent[e];
    const bool has_next = e + 1 < n;
    if (has_next) load_tile(int(ent[e + 1] >> 1));

    f32x16 s[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
      dp[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < C::DS; ++st) {
        const int off = (32 * kb + srow) * C::RST + 16 * st + 8 * hf;
        const u32x4 ak = *reinterpret_cast<const u32x4*>(&s_k[buf][off]);
        const u32x4 av = *reinterpret_cast<const u32x4*>(&s_v[buf][off]);
        s[kb] = mfma32x32x16<E>(ak, qf[st], s[kb]);
        dp[kb] = mfma32x32x16<E>(av, dof[st], dp[kb]);
      }
    }
    if (!(cur & 1u)) {
      const int k0 = int(cur >> 1) * C::BN;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int jl = 32 * kb + 16 * t + 8 * hf;
          const u32x4 c0 = *reinterpret_cast<const u32x4*>(&s_code[buf][jl]);
          const u32x4 c1 = *reinterpret_cast<const u32x4*>(&s_code[buf][jl + 4]);
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            const uint32_t kc = x < 4 ? c0[x] : c1[x - 4];
            if (!allow(qcode, kc, qrow, k0 + jl + x)) s[kb][8 * t + x] = NEG_INF;
          }
        }
      }
    }
    u32x4 dsb[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[kb][r], sl2, -lse));
        ds[r] = p * (dp[kb][r] - delta);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
        dsb[kb][t] = u32x4{pack2<E>(ds[8 * t + 0], ds[8 * t + 1]), pack2<E>(ds[8 * t + 2], ds[8 * t + 3]),
                           pack2<E>(ds[8 * t + 4], ds[8 * t + 5]), pack2<E>(ds[8 * t + 6], ds[8 * t + 7])};
    }
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const u32x4 ak = *reinterpret_cast<const u32x4*>(&s_kt[buf][(32 * db + c) * C::TST + 16 * t4 + 8 * hf]);
        acc[db] = mfma32x32x16<E>(ak, dsb[t4 >> 1][t4 & 1], acc[db]);
      }
    }
    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (qvalid) {
    uint16_t* g = static_cast<uint16_t*>(a.dq) + b * a.dq_strides[0] + h * a.dq_strides[1] + qrow * a.dq_strides[2];
    store_rows_T<E, D>(g, acc, a.sm_scale, hf);
  }
}

// ---------------------------------------------------------------- dK/dV ----
template <class E, int D>
__global__ __launch_bounds__(256) void k_dkdv(AttnArgs a, const uint32_t* __restrict__ codes,
                                              const uint32_t* __restrict__ list,
                                              const int32_t* __restrict__ count, int nT, int nKB) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t s_q[2][C::R_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_do[2][C::R_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_qt[2][C::T_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_dot[2][C::T_ELEMS];
  __shared__ __attribute__((aligned(16))) float s_lse[2][C::BN];
  __shared__ __attribute__((aligned(16))) float s_delta[2][C::BN];
  __shared__ __attribute__((aligned(16))) uint32_t s_code[2][C::BN];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / nKB;
  const int kblock = work % nKB;
  const int b = bh / H, h = bh % H;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* dog = static_cast<const uint16_t*>(a.dout) + b * a.do_strides[0] + h * a.do_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t* codes_b = codes + int64_t(b) * T;
  const float* lse_bh = a.lse + int64_t(bh) * T;
  const float* delta_bh = a.delta + int64_t(bh) * T;

  const int krow = kblock * 128 + wave * 32 + c;
  const bool kvalid = krow < T;
  u32x4 kf[C::DS], vf[C::DS];
#pragma unroll
  for (int st = 0; st < C::DS; ++st) {
    kf[st] = kvalid ? *reinterpret_cast<const u32x4*>(kg + krow * a.k_strides[2] + 16 * st + 8 * hf)
                    : u32x4{0, 0, 0, 0};
    vf[st] = kvalid ? *reinterpret_cast<const u32x4*>(vg + krow * a.v_strides[2] + 16 * st + 8 * hf)
                    : u32x4{0, 0, 0, 0};
  }
  const uint32_t kcode = kvalid ? codes_b[krow] : 0u;

  const int lbase = b * nKB + kblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  const float INF = __builtin_inff();
  u32x4 rq[4], rdo[4];
  float rsmall = 0.f;
  uint32_t rcode = 0;
  auto load_tile = [&](int qt) {
    const int q0 = qt * C::BN;
    if (tid < C::BLK) {
      load_block<D>(qg, a.q_strides[2], q0, T, tid, rq);
      load_block<D>(dog, a.do_strides[2], q0, T, tid, rdo);
    }
    const int x = tid & 63, qi = q0 + x;
    if (tid < 64) {
      float l = qi < T ? lse_bh[qi] : -INF;
      rsmall = (l == -INF) ? INF : l;
    } else if (tid < 128) {
      rsmall = qi < T ? delta_bh[qi] : 0.f;
    } else if (tid < 192) {
      rcode = qi < T ? codes_b[qi] : 0u;
    }
  };
  auto store_tile = [&](int buf) {
    if (tid < C::BLK) {
      store_block<D>(s_q[buf], s_qt[buf], tid, rq);
      store_block<D>(s_do[buf], s_dot[buf], tid, rdo);
    }
    const int x = tid & 63;
    if (tid < 64) s_lse[buf][x] = rsmall;
    else if (tid < 128) s_delta[buf][x] = rsmall;
    else if (tid < 192) s_code[buf][x] = rcode;
  };

  const float sl2 = a.sm_scale * 1.4426950408889634f;
  const float NEG_INF = -INF;
  f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  const int srow = sigma(c);

  if (n > 0) {
    load_tile(int(ent[0] >> 1));
    store_tile(0);
  }
  __syncthreads();

  for (int e = 0; e < n; ++e) {
    const int buf = e & 1;
    const uint32_t cur = ent[e];
    const bool has_next = e + 1 < n;
    if (has_next) load_tile(int(ent[e + 1] >> 1));
    const int q0 = int(cur >> 1) * C::BN;

#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int st = 0; st < C::DS; ++st) {
        const int off = (32 * qb + srow) * C::RST + 16 * st + 8 * hf;
        const u32x4 aq = *reinterpret_cast<const u32x4*>(&s_q[buf][off]);
        const u32x4 ao = *reinterpret_cast<const u32x4*>(&s_do[buf][off]);
        s = mfma32x32x16<E>(aq, kf[st], s);
        dp = mfma32x32x16<E>(ao, vf[st], dp);
      }
      // register r of s holds query 32*qb + 16*(r/8) + 8*hf + r%8, key = this lane's key
      u32x4 pb[2], dsb[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ql = 32 * qb + 16 * t + 8 * hf;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(&s_lse[buf][ql]);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(&s_lse[buf][ql + 4]);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(&s_delta[buf][ql]);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(&s_delta[buf][ql + 4]);
        u32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
        const bool partial = !(cur & 1u);
        if (partial) {
          c0 = *reinterpret_cast<const u32x4*>(&s_code[buf][ql]);
          c1 = *reinterpret_cast<const u32x4*>(&s_code[buf][ql + 4]);
        }
        float p[8], ds[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const float lx = x < 4 ? l0[x] : l1[x - 4];
          const float dx = x < 4 ? d0[x] : d1[x - 4];
          float sv = s[8 * t + x];
          if (partial) {
            const uint32_t qc = x < 4 ? c0[x] : c1[x - 4];
            if (!allow(qc, kcode, q0 + ql + x, krow)) sv = NEG_INF;
          }
          p[x] = fast_exp2(__builtin_fmaf(sv, sl2, -lx));
          ds[x] = p[x] * (dp[8 * t + x] - dx);
        }
        pb[t] = u32x4{pack2<E>(p[0], p[1]), pack2<E>(p[2], p[3]), pack2<E>(p[4], p[5]), pack2<E>(p[6], p[7])};
        dsb[t] = u32x4{pack2<E>(ds[0], ds[1]), pack2<E>(ds[2], ds[3]), pack2<E>(ds[4], ds[5]),
                       pack2<E>(ds[6], ds[7])};
      }
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int off = (32 * db + c) * C::TST + 16 * (2 * qb + t) + 8 * hf;
          const u32x4 ao = *reinterpret_cast<const u32x4*>(&s_dot[buf][off]);
          const u32x4 aq = *reinterpret_cast<const u32x4*>(&s_qt[buf][off]);
          dv[db] = mfma32x32x16<E>(ao, pb[t], dv[db]);
          dk[db] = mfma32x32x16<E>(aq, dsb[t], dk[db]);
        }
      }
    }
    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (kvalid) {
    uint16_t* gk = static_cast<uint16_t*>(a.dk) + b * a.dk_strides[0] + h * a.dk_strides[1] + krow * a.dk_strides[2];
    uint16_t* gv = static_cast<uint16_t*>(a.dv) + b * a.dv_strides[0] + h * a.dv_strides[1] + krow * a.dv_strides[2];
    store_rows_T<E, D>(gk, dk, a.sm_scale, hf);
    store_rows_T<E, D>(gv, dv, 1.f, hf);
  }
}

// -------------------------------------------------------------- launchers --
template <class E, int D>
static void launch_delta_t(const AttnArgs& a, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t rows = int64_t(a.B) * a.H * a.T;
  hipLaunchKernelGGL((k_delta<E, D>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, a);
}
template <class E, int D>
static void launch_dq_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const unsigned grid = unsigned(a.B) * a.H * L.n_dq_blocks;
  hipLaunchKernelGGL((k_dq<E, D>), dim3(grid), dim3(256), 0, st, a, reinterpret_cast<const uint32_t*>(plan + L.codes),
                     reinterpret_cast<const uint32_t*>(plan + L.dq_list),
                     reinterpret_cast<const int32_t*>(plan + L.dq_count), L.nT, L.n_dq_blocks);
}
template <class E, int D>
static void launch_dkdv_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const unsigned grid = unsigned(a.B) * a.H * L.n_dkdv_blocks;
  hipLaunchKernelGGL((k_dkdv<E, D>), dim3(grid), dim3(256), 0, st, a,
                     reinterpret_cast<const uint32_t*>(plan + L.codes),
                     reinterpret_cast<const uint32_t*>(plan + L.dkdv_list),
                     reinterpret_cast<const int32_t*>(plan + L.dkdv_count), L.nT, L.n_dkdv_blocks);
}

#define KD_DISPATCH(FN, ...)                                         \
  do {                                                               \
    if (a.dtype == KD_BF16) {                                        \
      if (a.D == 64) FN<BF16, 64>(__VA_ARGS__);                      \
      else FN<BF16, 128>(__VA_ARGS__);                               \
    } else {                                                         \
      if (a.D == 64) FN<F16, 64>(__VA_ARGS__);                       \
      else FN<F16, 128>(__VA_ARGS__);                                \
    }                                                                \
  } while (0)

int launch_delta(const AttnArgs& a, hipStream_t st) {
  KD_DISPATCH(launch_delta_t, a, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}
int launch_dq(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  KD_DISPATCH(launch_dq_t, a, plan, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}
int launch_dkdv(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  KD_DISPATCH(launch_dkdv_t, a, plan, st);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
