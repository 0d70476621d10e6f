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
// rescaled when a row's max grows by more than 2^R log2 units (rescale_log2),
// which removes the per-step O *= alpha of the textbook loop.  Without a
// rescale every P = exp2(S c - m_ref c) of the step is <= 2^R (up to the fp32
// rounding of the exponent, < 2^-10 absolute at |S c| < 2^13, and v_exp_f32's
// 1 ulp), and P is packed to the input type before P V:
//   bf16: R = 16, P <= 65536 (bf16 reaches 3.4e38; a high threshold rescales
//         less often than 2^8 on outlier data, -1%);
//   fp16: R = 15, P <= 32768 * (1 + 2^-9) < 65504, the fp16 maximum (R = 16
//         would round P in (65519.5, 65536] to +inf, and O to NaN).
// l and O stay far below the fp32 range over any row length.  Each wave masks by the class of its own 64-row q-tile
// against the key tile (from the list entry): FULL tiles skip the mask,
// PARTIAL ones build 64-bit row masks from the token codes (query_row_mask:
// a few wave ballots per tile) and apply them (two VALU ops per score),
// EMPTY ones mask everything.  O is normalised by the sum of the ROUNDED P that enters P V,
// so it is an exact convex combination of V rows up to the final rounding
// even when one key dominates the row; LSE uses the same sum.
#include "kd_tile.h"

namespace kd {

// largest log2 growth of a row's max that is absorbed without rescaling (see above)
template <class E> constexpr float rescale_log2();
template <> constexpr float rescale_log2<BF16>() { return 16.f; }
template <> constexpr float rescale_log2<F16>() { return 15.f; }

// LDS operand reads run this many MFMA steps ahead of their use: the K rows
// of the score product and the V^T blocks of P V
constexpr int FWD_PF = 4;

// NSP: the parts P enters P V in (1, 2 or 3: parts_of the precision)
template <class E, int D, bool Q8, int NSP>
__global__ __launch_bounds__(256, D <= 128 ? 2 : 1) void k_fwd(AttnArgs a, const uint32_t* __restrict__ codes,
                                                             const uint32_t* __restrict__ list,
                                                             const int32_t* __restrict__ count,
                                                             const uint32_t* __restrict__ order, int nT, int nQB) {
  constexpr bool SP = NSP >= 2, S3 = NSP == 3;
  constexpr int NW = 4;             // waves per 128-row q-block; each owns 32 rows
  using TL = Tile<D, NW>;           // V tiles (and K tiles on the 16-bit path)
  using SO = ScoreOp<E, D, Q8>;     // S^T = K Q^T, 16-bit or fp8
  using TK = Tile<Q8 ? D / 2 : D, NW>;  // K tiles (fp8: D bytes a row); same layout as SO::TL
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  constexpr int NL = TL::LOADS_PER_WAVE;
  constexpr int NLK = TK::LOADS_PER_WAVE;
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][TK::BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][TL::BYTES];
  // the token codes of each step's 64 keys (copied one step ahead by wave 0)
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[2][64];

  // the wave index through readfirstlane: uniform, so the role and slot
  // arithmetic derived from it stays scalar
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, hf = lane >> 5,
            c = lane & 31;
  const int T = a.T, H = a.H;
  int h, rank;  // (fwd_work: per XCD, the plan's longest-first order)
  fwd_work(blockIdx.x, gridDim.x, a.B * nQB, &h, &rank);
  const int item = int(order[rank]);
  const int b = item / nQB, qblock = item - b * nQB, bh = b * H + h;

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
  const u32x4 rs_k = rsrc_words(ks_base, uint32_t(T) * krb);
  const u32x4 rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  // bytes of a row of the 16-bit inputs: 2 D, or fewer for head dims 16 and
  // 32 on the D = 64 kernel, whose other columns are read as zeros
  const uint32_t dbytes = uint32_t(a.D) * 2u;

  // ---- this lane's query row (the B operand of S^T, kept in registers) ----
  const int srow = sigma(c);
  const int qrow = qblock * 128 + wave * 32 + c;
  const bool qvalid = qrow < T;
  SO so;
  so.load_b(rs_q, uint32_t(qrow) * qrb, hf, dbytes);
  so.init(srow, hf);
  // this wave's rows lie in q-tile 2 qblock + member of the block (group of 2)
  const int member = wave >> 1;
  // token codes of batch row b (reads past T return 0: allow nothing); the
  // row mask of a PARTIAL tile is built from them (query_row_mask)
  const u32x4 rs_codes = rsrc_words(codes + int64_t(b) * T, uint32_t(T) * 4u);
  uint32_t qcode = qvalid ? codes[int64_t(b) * T + qrow] : 0u;

  const int lbase = item;  // b nQB + qblock
  const int n = count[lbase];
  const uint32_t* ent = list + int64_t(lbase) * nT;

  uint32_t koff[NLK], voff[NL];
  TK::load_offsets(wave, lane, krb, koff, Q8 ? uint32_t(TK::ROWB) : dbytes);
  TL::load_offsets(wave, lane, vrb, voff, dbytes);
  // K tiles run one step ahead of V tiles (S of tile e+1 is computed while
  // tile e is softmaxed), so they are loaded separately.
  // slot = e & 1 (passed as a constant by the unrolled loop)
  auto load_k = [&](int e, int slot) {
    const uint32_t k0 = entry_tile(ent[e]) * 64u;
    TK::load_async(rs_k, k0 * krb, koff, lds_addr(s_k[slot]), wave);
  };
  auto load_v = [&](int e, int slot) {
    const uint32_t k0 = entry_tile(ent[e]) * 64u;
    TL::load_async(rs_v, k0 * vrb, voff, lds_addr(s_v[slot]), wave);
  };
  // the 64 key codes of tile e, copied to LDS one step ahead of their use
  // by wave 0 (a register load would be waited for by the compiler, together
  // with the tile copies after it)
  auto load_codes = [&](int e, int slot) {
    if (wave == 0)
      dma_b32(rs_codes, (entry_tile(ent[e]) * 64u + uint32_t(lane)) * 4u,
              uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(&s_kc[slot][0])))));
  };

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
  // S^T = K Q^T for one tile: two 32-key halves.  The K operand of k-step i
  // is read FWD_PF steps before its MFMA; the sched_barriers keep LDS reads
  // and MFMAs in this order (VALU, SALU and transcendental work may move
  // across them, to fill the MFMA shadow).
  auto scores = [&](const uint8_t* kt, f32x16 (&s)[2]) {
    constexpr int NS = 2 * SO::NK, PF = FWD_PF < NS ? FWD_PF : NS;  // steps: kb = i & 1, st = i >> 1
    typename SO::A av[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) av[i] = so.read_a(kt, i & 1, i >> 1);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int kb = i & 1, st = i >> 1;
      __builtin_amdgcn_sched_barrier(0x406);
      s[kb] = so.mma_a(av[i % PF], st, st == 0 ? f32x16{} : s[kb]);
      if (i + PF < NS) av[i % PF] = so.read_a(kt, (i + PF) & 1, (i + PF) >> 1);
    }
    __builtin_amdgcn_sched_barrier(0x406);
  };

  // the fp8 product carries the dequantisation scales of Q and K
  const float sl2 = a.sm_scale * 1.4426950408889634f * (Q8 ? a.q_scale[bh] * a.k_scale[bh] : 1.f);
  const float NEG_INF = -__builtin_inff();
  float m_ref = NEG_INF, l0 = 0.f, l1 = 0.f;
  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};

  f32x16 s[2];
  if (n > 0) {
    load_k(0, 0);
    load_v(0, 0);
    if (n > 1) load_k(1, 1);
    load_codes(0, 0);
    wait_vmem();
    so.settle();  // the compiler's wait for the Q rows (and query codes) falls here
    settle(qcode);
    __syncthreads();
    scores(s_k[0], s);
  }

  // One step per key tile; unrolled by two so that the buffer of each step is
  // a constant and every LDS address is a fixed register plus an immediate.
  auto step = [&](const int e, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;  // == e & 1
    const uint32_t cur = ent[e];
    // The tile copies are inline asm (see dma_b128), so the compiler sees no
    // load in flight and places no wait of its own before the LDS reads of
    // this step: the copies issued below stay in flight for the whole step.
    wait_vmem();
    barrier_raw();  // V(e), K(e+1) and the masks landed; every wave is done with K(e) and V(e-1)
    if (e + 1 < n) {
      load_v(e + 1, buf ^ 1);
      load_codes(e + 1, buf ^ 1);
    }
    if (e + 2 < n) load_k(e + 2, buf);

    const uint32_t mcls = entry_class(cur, member);
    if (mcls != TILE_FULL) {  // wave-uniform.  Register r of s[kb] holds key 32 kb + 16 (r / 8) + 8 hf + r % 8
      // of the tile: bit 16 (r / 8) + r % 8 of word kb of the row mask shifted by 8 hf
      const uint64_t rowbits = mcls == TILE_PARTIAL  // EMPTY: nothing allowed
                                   ? query_row_mask(qcode, qrow, s_kc[buf][lane], int(entry_tile(cur)) * 64)
                                   : 0u;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const uint32_t w = uint32_t(rowbits >> (32 * kb)) >> (8 * hf);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = mask_bit(s[kb][r], w, 16 * (r >> 3) + (r & 7));
      }
    }
    // running max of this lane's row; rescale only when it grows by > rescale_log2 (P bound)
    float ms;
    {
      float mx = NEG_INF;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = xhalf_max(mx);
      const float m_new = fmaxf(m_ref, mx);
      if ((m_new - m_ref) * sl2 > rescale_log2<E>()) {  // false for -inf - -inf (NaN); per lane
        const float alpha = (m_ref == NEG_INF) ? 0.f : fast_exp2((m_ref - m_new) * sl2);
        m_ref = m_new;
        l0 *= alpha;
        l1 *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
      }
      ms = (m_ref == NEG_INF) ? 0.f : m_ref * sl2;
    }

    // softmax of tile e (VALU) alongside S of tile e+1 (MFMA; computed from
    // the other K buffer even past the last tile, where it is simply unused)
    // P packed for the MFMA (pk) and, with SP, its rounding residual (pl):
    // P V is then formed as pk V + pl V, P carried to ~16 significant bits;
    // with S3 a third part pm carries it to ~24
    u32x4 pk[2][2];
    u32x4 pl[2][2];
    u32x4 pm[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(__builtin_fmaf(s[kb][r], sl2, -ms));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pk[kb][t] = pack8<E>(p + 8 * t);
        l0 = acc_pair<E>(pk[kb][t][0], l0);
        l1 = acc_pair<E>(pk[kb][t][1], l1);
        l0 = acc_pair<E>(pk[kb][t][2], l0);
        l1 = acc_pair<E>(pk[kb][t][3], l1);
        if constexpr (SP) {
          pl[kb][t] = pack8_residual<E>(p + 8 * t, pk[kb][t]);
          l0 = acc_pair<E>(pl[kb][t][0], l0);
          l1 = acc_pair<E>(pl[kb][t][1], l1);
          l0 = acc_pair<E>(pl[kb][t][2], l0);
          l1 = acc_pair<E>(pl[kb][t][3], l1);
        }
        if constexpr (S3) {
          pm[kb][t] = pack8_residual2<E>(p + 8 * t, pk[kb][t], pl[kb][t]);
          l0 = acc_pair<E>(pm[kb][t][0], l0);
          l1 = acc_pair<E>(pm[kb][t][1], l1);
          l0 = acc_pair<E>(pm[kb][t][2], l0);
          l1 = acc_pair<E>(pm[kb][t][3], l1);
        }
      }
    }
    scores(s_k[buf ^ 1], s);
    // O^T += V^T P^T for tile e, each V^T operand read FWD_PF steps ahead of
    // its MFMA (steps: t4 = i / DB, db = i % DB)
    const uint8_t* vt = s_v[buf];
    {
      constexpr int NV = 4 * DB, PFV = FWD_PF < NV ? FWD_PF : NV;
      auto read_v = [&](int i) {
        const int t4 = i / DB, db = i % DB;
        const u32x2 lo = ds_read_tr16(vt + vaddr[db][0] + t4 * 16 * TL::ROWB);
        const u32x2 hi = ds_read_tr16(vt + vaddr[db][1] + t4 * 16 * TL::ROWB);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vv[PFV];
#pragma unroll
      for (int i = 0; i < PFV; ++i) vv[i] = read_v(i);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int t4 = i / DB, db = i % DB;
        __builtin_amdgcn_sched_barrier(0x406);
        o[db] = mfma32x32x16<E>(vv[i % PFV], pk[t4 >> 1][t4 & 1], o[db]);
        if constexpr (SP) o[db] = mfma32x32x16<E>(vv[i % PFV], pl[t4 >> 1][t4 & 1], o[db]);
        if constexpr (S3) o[db] = mfma32x32x16<E>(vv[i % PFV], pm[t4 >> 1][t4 & 1], o[db]);
        if (i + PFV < NV) vv[i % PFV] = read_v(i + PFV);
      }
      __builtin_amdgcn_sched_barrier(0x406);
    }
  };
  for (int e = 0; e < n; e += 2) {
    step(e, std::integral_constant<int, 0>{});
    if (e + 1 < n) step(e + 1, std::integral_constant<int, 1>{});
  }

  // ---- epilogue: normalise, store O and LSE ----
  // O and LSE use the row sum of the ROUNDED P that entered P V (summed two
  // at a time by v_dot2c): O's weights then sum to exactly 1, and the sum
  // costs half an instruction per score instead of one fp32 add
  {
    const float l_tot = xhalf_sum(l0 + l1);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qvalid) {
      const int row = qrow;
      uint16_t* og = static_cast<uint16_t*>(a.o) + b * a.o_strides[0] + h * a.o_strides[1] + row * a.o_strides[2];
      // optional rounding residual O - bf16(O), so the backward's Delta can be
      // formed from O to ~16 significant bits (contiguous [B, H, T, a.D]); in
      // fp32 with S3, so that O + O_lo is the fp32 O
      uint16_t* lg = a.o_lo == nullptr || S3 ? nullptr
                                             : static_cast<uint16_t*>(a.o_lo) + (int64_t(bh) * T + row) * a.D;
      float* lg32 = a.o_lo == nullptr || !S3 ? nullptr
                                             : static_cast<float*>(a.o_lo) + (int64_t(bh) * T + row) * a.D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * db + 8 * g + 4 * hf;
          if (D == 64 && d0 >= a.D) continue;  // head dims 16, 32: only the real columns
          float f[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) f[i] = o[db][4 * g + i] * inv;
          const u32x2 w = {pack2<E>(f[0], f[1]), pack2<E>(f[2], f[3])};
          *reinterpret_cast<u32x2*>(og + d0) = w;
          if (lg != nullptr) {
            const u32x2 r = {pack2_residual<E>(f[0], f[1], w[0]), pack2_residual<E>(f[2], f[3], w[1])};
            *reinterpret_cast<u32x2*>(lg + d0) = r;
          }
          if (lg32 != nullptr)
            *reinterpret_cast<f32x4*>(lg32 + d0) =
                f32x4{f[0] - to_f32<E>(uint16_t(w[0] & 0xFFFFu)), f[1] - to_f32<E>(uint16_t(w[0] >> 16)),
                      f[2] - to_f32<E>(uint16_t(w[1] & 0xFFFFu)), f[3] - to_f32<E>(uint16_t(w[1] >> 16))};
        }
      }
      if (a.lse != nullptr && hf == 0)
        a.lse[int64_t(bh) * T + row] = l_tot > 0.f ? m_ref * sl2 + fast_log2(l_tot) : NEG_INF;
    }
  }
}

template <class E, int D, bool Q8, int NSP>
static void launch_fwd_t(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const int nQB = L.n_fwd_blocks;
  const unsigned grid = unsigned(a.B) * a.H * nQB;
  hipLaunchKernelGGL((k_fwd<E, D, Q8, NSP>), dim3(grid), dim3(256), 0, st, a,
                     reinterpret_cast<const uint32_t*>(plan + L.codes),
                     reinterpret_cast<const uint32_t*>(plan + L.fwd_list),
                     reinterpret_cast<const int32_t*>(plan + L.fwd_count),
                     reinterpret_cast<const uint32_t*>(plan + L.fwd_order), L.nT, nQB);
}

template <class E, int D, bool Q8 = false>
static void launch_fwd_p(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  switch (parts_of(a.precision)) {
    case 1: launch_fwd_t<E, D, Q8, 1>(a, plan, st); break;
    case 2: launch_fwd_t<E, D, Q8, 2>(a, plan, st); break;
    default:
      if constexpr (!Q8) launch_fwd_t<E, D, Q8, 3>(a, plan, st);  // (the C ABI refuses it with fp8 scores)
      break;
  }
}

int launch_fwd(const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  if (use_simt(a)) return launch_simt_kernel(0, a, plan, st);
  if (a.q8 != nullptr) {  // fp8 QK^T: bf16 at head dim 64, 128 or 256 (checked by the C ABI)
    if (a.D == 64) launch_fwd_p<BF16, 64, true>(a, plan, st);
    else if (a.D == 128) launch_fwd_p<BF16, 128, true>(a, plan, st);
    else launch_fwd_p<BF16, 256, true>(a, plan, st);
  } else if (a.dtype == KD_BF16) {  // head dims 16 and 32 on the D = 64 kernel
    if (a.D <= 64) launch_fwd_p<BF16, 64>(a, plan, st);
    else if (a.D == 128) launch_fwd_p<BF16, 128>(a, plan, st);
    else launch_fwd_p<BF16, 256>(a, plan, st);
  } else {
    if (a.D <= 64) launch_fwd_p<F16, 64>(a, plan, st);
    else if (a.D == 128) launch_fwd_p<F16, 128>(a, plan, st);
    else launch_fwd_p<F16, 256>(a, plan, st);
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
