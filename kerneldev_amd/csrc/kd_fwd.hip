// Forward hierarchical-mask flash attention on gfx950 bf16/fp16 MFMA.
//
// Computes what _flash_attn_fwd does (original_kernel.py:279-626): per query
// row, O = softmax2(S * c) V over the allowed keys and LSE2 = m + log2(l),
// with c = sm_scale * log2(e) kept in fp32 (the reference rounds it to the
// input dtype at :415; deliberately not reproduced).
//
// Layout per workgroup: 4 waves x 32 query rows = 128 rows (one q-block of
// the plan's forward list), 64 keys per step.  Each wave computes
//   S^T[64 keys x 32 q]  = K Q^T      (A = K rows from LDS, B = Q in registers)
//   O^T[D x 32 q]       += V^T P^T    (A = V^T from LDS,   B = P in registers)
// so a lane owns one query column: the softmax row statistics are per-lane
// scalars (one cross-half max per step), and P never leaves registers thanks
// to the sigma() row permutation of the K operand.  K and V^T tiles are
// double buffered in LDS; the next tile's global loads are in flight while
// the current one is computed.  Only non-empty key tiles are visited (plan
// list); FULL tiles skip the mask, PARTIAL tiles evaluate it per element.
#include "kd_internal.h"

namespace kd {

template <int D>
struct FwdCfg {
  static constexpr int BN = 64;              // keys per step
  static constexpr int KST = D + 8;          // K row stride (elements) in LDS
  static constexpr int VST = BN + 8;         // V^T row stride (elements) in LDS
  static constexpr int DS = D / 16;          // 16-wide k-steps over d
  static constexpr int DB = D / 32;          // 32-row blocks of O^T
  static constexpr int KCH = BN * D / 8 / 256;  // 16-byte K chunks per thread
  static constexpr int VBLK = (BN / 4) * (D / 8);  // 4-key x 8-d V blocks
  static constexpr int K_ELEMS = BN * KST;
  static constexpr int V_ELEMS = D * VST;
};

template <class E, int D>
__global__ __launch_bounds__(256) void k_fwd(AttnArgs a, const uint32_t* __restrict__ codes,
                                             const uint32_t* __restrict__ list,
                                             const int32_t* __restrict__ count, int nT, int nQB) {
  using C = FwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t s_k[2][C::K_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t s_vt[2][C::V_ELEMS];
  __shared__ __attribute__((aligned(16))) uint32_t s_code[2][C::BN];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / nQB;
  const int qblock = nQB - 1 - (work % nQB);  // heaviest (latest) q-blocks first
  const int b = bh / H, h = bh % H;

  const uint16_t* qg = static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] + h * a.q_strides[1];
  const uint16_t* kg = static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] + h * a.k_strides[1];
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const int64_t kst = a.k_strides[2], vst = a.v_strides[2];
  const uint32_t* codes_b = codes + int64_t(b) * T;

  // ---- per-lane query row ----
  const int qrow = qblock * 128 + wave * 32 + c;
  const bool qvalid = qrow < T;
  u32x4 qf[C::DS];
#pragma unroll
  for (int st = 0; st < C::DS; ++st) {
    qf[st] = qvalid ? *reinterpret_cast<const u32x4*>(qg + qrow * a.q_strides[2] + 16 * st + 8 * hf)
                    : u32x4{0, 0, 0, 0};
  }
  const uint32_t qcode = qvalid ? codes_b[qrow] : 0u;

  const int lbase = b * nQB + qblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  // ---- tile loader: global -> registers -> LDS ----
  u32x4 rk[C::KCH];
  u32x4 rv[4];
  uint32_t rcode = 0;
  auto load_tile = [&](int kt) {
    const int k0 = kt * C::BN;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int ch = tid + 256 * i, row = ch / (D / 8), col = ch % (D / 8);
      const int key = k0 + row;
      rk[i] = key < T ? *reinterpret_cast<const u32x4*>(kg + key * kst + col * 8) : u32x4{0, 0, 0, 0};
    }
    if (tid < C::VBLK) {
      const int kgp = tid / (D / 8), dc = tid % (D / 8);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 4 * kgp + r;
        rv[r] = key < T ? *reinterpret_cast<const u32x4*>(vg + key * vst + dc * 8) : u32x4{0, 0, 0, 0};
      }
    }
    if (tid < C::BN) rcode = (k0 + tid < T) ? codes_b[k0 + tid] : 0u;
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int ch = tid + 256 * i, row = ch / (D / 8), col = ch % (D / 8);
      *reinterpret_cast<u32x4*>(&s_k[buf][row * C::KST + col * 8]) = rk[i];
    }
    if (tid < C::VBLK) {
      const int kgp = tid / (D / 8), dc = tid % (D / 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        u32x2 lo = {pack_lo(rv[0][w], rv[1][w]), pack_lo(rv[2][w], rv[3][w])};
        u32x2 hi = {pack_hi(rv[0][w], rv[1][w]), pack_hi(rv[2][w], rv[3][w])};
        *reinterpret_cast<u32x2*>(&s_vt[buf][(8 * dc + 2 * w) * C::VST + 4 * kgp]) = lo;
        *reinterpret_cast<u32x2*>(&s_vt[buf][(8 * dc + 2 * w + 1) * C::VST + 4 * kgp]) = hi;
      }
    }
    if (tid < C::BN) s_code[buf][tid] = rcode;
  };

  const float sl2 = a.sm_scale * 1.4426950408889634f;
  const float NEG_INF = -__builtin_inff();
  float m_i = NEG_INF, l_i = 0.f;
  f32x16 o[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) o[db] = f32x16{};

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

    // S^T = K Q^T for two 32-key blocks
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < C::DS; ++st) {
        const u32x4 ak = *reinterpret_cast<const u32x4*>(&s_k[buf][(32 * kb + srow) * C::KST + 16 * st + 8 * hf]);
        s[kb] = mfma32x32x16<E>(ak, qf[st], s[kb]);
      }
    }
    if (!(cur & 1u)) {  // PARTIAL tile: evaluate the mask per element
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
    // online softmax (base 2); statistics are per query = per lane column
    float mx = NEG_INF;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = wave_max32(mx);
    const float m_new = fmaxf(m_i, mx);
    const float ms = (m_new == NEG_INF) ? 0.f : m_new * sl2;
    const float alpha = fast_exp2(m_i * sl2 - ms);
    m_i = m_new;
    u32x4 pk[2][2];
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(__builtin_fmaf(s[kb][r], sl2, -ms));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pk[kb][t] = u32x4{pack2<E>(p[8 * t + 0], p[8 * t + 1]), pack2<E>(p[8 * t + 2], p[8 * t + 3]),
                          pack2<E>(p[8 * t + 4], p[8 * t + 5]), pack2<E>(p[8 * t + 6], p[8 * t + 7])};
        // the row sum uses the ROUNDED P that enters P V, so O = sum(P V) / sum(P)
        // is a convex combination of V rows even when one key dominates
#pragma unroll
        for (int w = 0; w < 4; ++w) lsum += sum2<E>(pk[kb][t][w]);
      }
    }
    l_i = l_i * alpha + lsum;
#pragma unroll
    for (int db = 0; db < C::DB; ++db) o[db] *= alpha;
    // O^T += V^T P^T
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(&s_vt[buf][(32 * db + c) * C::VST + 16 * t4 + 8 * hf]);
        o[db] = mfma32x32x16<E>(av, pk[t4 >> 1][t4 & 1], o[db]);
      }
    }
    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, store O and LSE ----
  const float l_tot = wave_sum32(l_i);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qvalid) {
    uint16_t* og = static_cast<uint16_t*>(a.o) + b * a.o_strides[0] + h * a.o_strides[1] + qrow * a.o_strides[2];
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * hf;
        u32x2 w = {pack2<E>(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                   pack2<E>(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2*>(og + d0) = w;
      }
    }
    if (a.lse != nullptr && hf == 0)
      a.lse[int64_t(bh) * T + qrow] = l_tot > 0.f ? m_i * sl2 + fast_log2(l_tot) : NEG_INF;
  }
}

template <class E, int D>
static void launch_fwd_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const int nQB = L.n_fwd_blocks;
  const unsigned grid = unsigned(a.B) * a.H * nQB;
  hipLaunchKernelGGL((k_fwd<E, D>), dim3(grid), dim3(256), 0, st, a,
                     reinterpret_cast<const uint32_t*>(plan + L.codes),
                     reinterpret_cast<const uint32_t*>(plan + L.fwd_list),
                     reinterpret_cast<const int32_t*>(plan + L.fwd_count), L.nT, nQB);
}

int launch_fwd(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (a.dtype == KD_BF16) {
    if (a.D == 64) launch_fwd_t<BF16, 64>(a, plan, st);
    else launch_fwd_t<BF16, 128>(a, plan, st);
  } else {
    if (a.D == 64) launch_fwd_t<F16, 64>(a, plan, st);
    else launch_fwd_t<F16, 128>(a, plan, st);
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
