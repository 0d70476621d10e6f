// Forward hierarchical-mask flash attention on gfx950 bf16/fp16 MFMA.
//
// Computes what _flash_attn_fwd does (original_kernel.py:279-626): per query
// row, O = softmax2(S * c) V over the allowed keys and LSE2 = m + log2(l),
// with c = sm_scale * log2(e) kept in fp32 (the reference rounds it to the
// input dtype at :415; deliberately not reproduced).
//
// One workgroup = 4 waves x 32 query rows = one 128-row q-block of the plan's
// forward list; 64 keys per step.  Each wave computes
//   S^T[64 keys x 32 q]  = K Q^T      (A = K rows from LDS, B = Q in registers)
//   O^T[D x 32 q]       += V^T P^T    (A = V^T read transposed from LDS,
//                                      B = P straight from the S^T registers)
// so a lane owns one query column: the softmax statistics are per-lane
// scalars plus one permlane32 exchange, and P never leaves registers thanks to
// the sigma() row permutation of the K operand.  K and V tiles are copied
// global -> LDS by buffer_load ... lds and V is transposed by ds_read_b64_tr_b16
// on the way into the MFMA.  The loop is software pipelined: while the
// softmax of tile e runs on the VALU, the MFMAs already compute S of tile
// e+1 (K tiles are loaded one step ahead of V tiles, both double buffered).  Only non-empty key tiles are
// visited (plan list); FULL tiles skip the mask, PARTIAL tiles evaluate it.
//
// The running max is rescaled lazily, per lane: the accumulators are only
// rescaled when a row's max grows by more than 2^8 (P is then <= 256,
// harmless in fp32/bf16), which removes the per-step O *= alpha of the
// textbook loop.  PARTIAL tiles are masked with the table form of the rule
// (kd_common.h: qmask / mask_score), a handful of VALU ops per score.
// O is normalised by the sum of the ROUNDED P that enters P V, so it is an
// exact convex combination of V rows up to the final rounding even when one
// key dominates the row; LSE uses the exact fp32 sum.
#include "kd_tile.h"

namespace kd {

template <class E, int D, bool Q8>
__global__ __launch_bounds__(256, 2) void k_fwd(AttnArgs a, const uint32_t* __restrict__ codes,
                                                const uint32_t* __restrict__ list,
                                                const int32_t* __restrict__ count, int nT, int nQB) {
  using TL = Tile<D>;           // V tiles (and K tiles on the 16-bit path)
  using SO = ScoreOp<E, D, Q8>;  // S^T = K Q^T, 16-bit or fp8
  using TK = typename SO::TL;   // K tiles
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  constexpr int NL = TL::LOADS_PER_WAVE;
  constexpr int NLK = TK::LOADS_PER_WAVE;
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][TK::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][TL::BYTES];
  __shared__ __attribute__((aligned(256))) uint32_t s_code[2][64];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, c = lane & 31;
  const int T = a.T, H = a.H;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int hb = work / nQB;  // head-major: each XCD's range holds every batch row of its heads
  const int qblock = nQB - 1 - (work % nQB);  // heaviest (latest) q-blocks first
  const int b = hb % a.B, h = hb / a.B, bh = b * H + h;

  // Q and K as the score product sees them: the 16-bit inputs, or their
  // contiguous fp8 copies (kd_quant_fp8)
  const void* qs_base = Q8 ? static_cast<const void*>(a.q8 + int64_t(bh) * T * D)
                           : static_cast<const void*>(static_cast<const uint16_t*>(a.q) + b * a.q_strides[0] +
                                                      h * a.q_strides[1]);
  const void* ks_base = Q8 ? static_cast<const void*>(a.k8 + int64_t(bh) * T * D)
                           : static_cast<const void*>(static_cast<const uint16_t*>(a.k) + b * a.k_strides[0] +
                                                      h * a.k_strides[1]);
  const uint32_t qrb = Q8 ? uint32_t(D) : uint32_t(a.q_strides[2]) * 2u;
  const uint32_t krb = Q8 ? uint32_t(D) : uint32_t(a.k_strides[2]) * 2u;
  const uint16_t* vg = static_cast<const uint16_t*>(a.v) + b * a.v_strides[0] + h * a.v_strides[1];
  const uint32_t vrb = uint32_t(a.v_strides[2]) * 2u;
  const auto rs_q = make_rsrc(qs_base, uint32_t(T) * qrb);
  const auto rs_k = make_rsrc(ks_base, uint32_t(T) * krb);
  const auto rs_v = make_rsrc(vg, uint32_t(T) * vrb);
  const auto rs_c = make_rsrc(codes + int64_t(b) * T, uint32_t(T) * 4u);

  // ---- per-lane query row (B operand of S^T, kept in registers) ----
  const int qrow = qblock * 128 + wave * 32 + c;
  const bool qvalid = qrow < T;
  SO so;
  so.load_b(rs_q, uint32_t(qrow) * qrb, hf);
  const uint32_t qcode = qvalid ? codes[int64_t(b) * T + qrow] : 0u;

  const int lbase = b * nQB + qblock;
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  uint32_t koff[NLK], voff[NL];
  TK::load_offsets(wave, lane, krb, koff);
  TL::load_offsets(wave, lane, vrb, voff);
  // K tiles run one step ahead of V tiles (S of tile e+1 is computed while
  // tile e is softmaxed), so they are loaded separately; the key codes of a
  // tile travel with its V tile.
  auto load_k = [&](int e) {
    const uint32_t k0 = uint32_t(ent[e] >> 1) * 64u;
    TK::load(rs_k, k0 * krb, koff, s_k[e & 1], wave);
  };
  auto load_v = [&](int e) {
    const uint32_t k0 = uint32_t(ent[e] >> 1) * 64u;
    TL::load(rs_v, k0 * vrb, voff, s_v[e & 1], wave);
    if (wave == 0)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_c, (lds_t*)&s_code[e & 1][0], 4, (k0 + lane) * 4u, 0, 0, 0);
  };

  // ---- LDS read addresses (bytes within a tile) ----
  // K operand: row 32 kb + sigma(c), this lane's k-slots of each k-step
  const int srow = sigma(c);
  so.init(srow, hf);
  // V^T operand via transposed reads: group g = lane / 16 covers d columns
  // 32 db + 16 (g & 1) .. +15 and key rows 16 t4 + 8 (g >> 1) + 4 half .. +3
  int vaddr[DB][2];
  {
    const int i = lane & 15, g = lane >> 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r = 8 * (g >> 1) + 4 * half + (i >> 2);
        const int chunk = 4 * db + 2 * (g & 1) + ((i & 3) >> 1);
        vaddr[db][half] = TL::at(r, chunk) + 8 * (i & 1);
      }
  }
  // S^T = K Q^T for one tile (two 32-key halves, independent chains)
  auto scores = [&](const uint8_t* kt, f32x16 (&s)[2]) {
    s[0] = f32x16{};
    s[1] = f32x16{};
    so.mma(kt, 0, s[0]);
    so.mma(kt, 1, s[1]);
  };

  // the fp8 product carries the dequantisation scales of Q and K
  const float sl2 = a.sm_scale * 1.4426950408889634f * (Q8 ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
  const float NEG_INF = -__builtin_inff();
  float m_ref = NEG_INF, l0 = 0.f, l1 = 0.f, le0 = 0.f, le1 = 0.f;
  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  const MaskTab mt = qmask(qcode);
  const int i_lo = qblock * 128 + wave * 32;  // this wave's query rows: i_lo .. i_lo + 31

  f32x16 s[2] = {f32x16{}, f32x16{}};
  if (n > 0) {
    load_k(0);
    load_v(0);
    if (n > 1) load_k(1);
    wait_vmem();
    __syncthreads();
    scores(s_k[0], s);
  }

  for (int e = 0; e < n; ++e) {
    const int buf = e & 1;
    const uint32_t cur = ent[e];
    wait_vmem();
    __syncthreads();  // V(e) and K(e+1) landed; every wave is done with K(e) and V(e-1)
    if (e + 1 < n) load_v(e + 1);
    if (e + 2 < n) load_k(e + 2);
    const int k0 = int(cur >> 1) * 64;

    if (!(cur & 1u)) {  // PARTIAL tile: register r of s[kb] holds key k0 + 32 kb + 16 (r / 8) + 8 hf + r % 8
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int j0 = k0 + 32 * kb;
        const bool below = j0 + 31 <= i_lo, above = j0 > i_lo + 31;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int jl = 32 * kb + 16 * t + 8 * hf;
          const u32x4 c0 = *reinterpret_cast<const u32x4*>(&s_code[buf][jl]);
          const u32x4 c1 = *reinterpret_cast<const u32x4*>(&s_code[buf][jl + 4]);
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            const uint32_t kc = x < 4 ? c0[x] : c1[x - 4];
            uint32_t tbl = below ? mt.hi : mt.lo;
            if (!below && !above) tbl = (k0 + jl + x <= qrow) ? mt.hi : mt.lo;
            s[kb][8 * t + x] = mask_score(s[kb][8 * t + x], tbl, kc, kc, mt.rsh);
          }
        }
      }
    }
    // running max of this lane's row; rescale only when it grows by > 2^8
    float mx = NEG_INF;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m_ref, mx);
    if ((m_new - m_ref) * sl2 > 8.f) {  // false for -inf - -inf (NaN); per lane
      const float alpha = (m_ref == NEG_INF) ? 0.f : fast_exp2((m_ref - m_new) * sl2);
      m_ref = m_new;
      l0 *= alpha;
      l1 *= alpha;
      le0 *= alpha;
      le1 *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
    }
    const float ms = (m_ref == NEG_INF) ? 0.f : m_ref * sl2;

    // softmax of tile e (VALU) alongside S of tile e+1 (MFMA; computed from
    // the other K buffer even past the last tile, where it is simply unused)
    u32x4 pk[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(__builtin_fmaf(s[kb][r], sl2, -ms));
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        le0 += p[r];
        le1 += p[r + 1];
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pk[kb][t] = u32x4{pack2<E>(p[8 * t + 0], p[8 * t + 1]), pack2<E>(p[8 * t + 2], p[8 * t + 3]),
                          pack2<E>(p[8 * t + 4], p[8 * t + 5]), pack2<E>(p[8 * t + 6], p[8 * t + 7])};
        l0 = acc_pair<E>(pk[kb][t][0], l0);
        l1 = acc_pair<E>(pk[kb][t][1], l1);
        l0 = acc_pair<E>(pk[kb][t][2], l0);
        l1 = acc_pair<E>(pk[kb][t][3], l1);
      }
    }
    scores(s_k[buf ^ 1], s);
    // O^T += V^T P^T for tile e
    const uint8_t* vt = s_v[buf];
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 lo = ds_read_tr16(vt + vaddr[db][0] + t4 * 16 * TL::ROWB);
        const u32x2 hi = ds_read_tr16(vt + vaddr[db][1] + t4 * 16 * TL::ROWB);
        o[db] = mfma32x32x16<E>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[t4 >> 1][t4 & 1], o[db]);
      }
    }
  }

  // ---- epilogue: normalise, store O and LSE ----
  // O is normalised by the sum of the ROUNDED P that entered P V (exact
  // convex weights); LSE by the exact fp32 sum, which is what the backward's
  // recomputed P = exp2(S c - LSE) must sum to
  const float l_tot = xhalf_sum(l0 + l1);
  const float l_exact = xhalf_sum(le0 + le1);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qvalid) {
    uint16_t* og = static_cast<uint16_t*>(a.o) + b * a.o_strides[0] + h * a.o_strides[1] + qrow * a.o_strides[2];
    // optional rounding residual O - bf16(O), so the backward's Delta can be
    // formed from O to ~16 significant bits (contiguous [B, H, T, D])
    uint16_t* lg = a.o_lo == nullptr ? nullptr
                                     : static_cast<uint16_t*>(a.o_lo) + (int64_t(bh) * T + qrow) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * hf;
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = o[db][4 * g + i] * inv;
        const u32x2 w = {pack2<E>(f[0], f[1]), pack2<E>(f[2], f[3])};
        *reinterpret_cast<u32x2*>(og + d0) = w;
        if (lg != nullptr) {
          const u32x2 r = {pack2<E>(f[0] - to_f32<E>(uint16_t(w[0] & 0xFFFFu)), f[1] - to_f32<E>(uint16_t(w[0] >> 16))),
                           pack2<E>(f[2] - to_f32<E>(uint16_t(w[1] & 0xFFFFu)), f[3] - to_f32<E>(uint16_t(w[1] >> 16)))};
          *reinterpret_cast<u32x2*>(lg + d0) = r;
        }
      }
    }
    if (a.lse != nullptr && hf == 0)
      a.lse[int64_t(bh) * T + qrow] = l_exact > 0.f ? m_ref * sl2 + fast_log2(l_exact) : NEG_INF;
  }
}

template <class E, int D, bool Q8 = false>
static void launch_fwd_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const int nQB = L.n_fwd_blocks;
  const unsigned grid = unsigned(a.B) * a.H * nQB;
  hipLaunchKernelGGL((k_fwd<E, D, Q8>), dim3(grid), dim3(256), 0, st, a,
                     reinterpret_cast<const uint32_t*>(plan + L.codes),
                     reinterpret_cast<const uint32_t*>(plan + L.fwd_list),
                     reinterpret_cast<const int32_t*>(plan + L.fwd_count), L.nT, nQB);
}

int launch_fwd(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (a.q8 != nullptr) {  // fp8 QK^T: bf16, head dim 128 (checked by the C ABI)
    launch_fwd_t<BF16, 128, true>(a, plan, st);
  } else if (a.dtype == KD_BF16) {
    if (a.D == 64) launch_fwd_t<BF16, 64>(a, plan, st);
    else launch_fwd_t<BF16, 128>(a, plan, st);
  } else {
    if (a.D == 64) launch_fwd_t<F16, 64>(a, plan, st);
    else launch_fwd_t<F16, 128>(a, plan, st);
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
