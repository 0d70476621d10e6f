// Attention for fp32 inputs on the fp32 matrix cores in their 16 x 16 x 4
// form (v_mfma_f32_16x16x4f32), for head dims WD = 32, 64, 128 and 256 (16
// is zero-padded to 32 by the Python layer): the reference's fp32 dots
// (original_kernel.py:452, :569, :1239, :1331-1333, :1425, :1517-1523) for
// HEAD_DIM in {32, 64, 128, 256} (:1720), fp32 operands and fp32
// accumulation.  Same algebra, plan, lists and masks as the 16-bit kernels:
//   forward   O = softmax2(S c) V, LSE2 = m + log2 l      (:279-626)
//   dQ        P = exp2(S c - LSE), dS = P (dP - Delta), dQ = sm_scale dS K  (:1173-1336)
//   dK / dV   dV = P^T dO, dK = sm_scale dS^T Q            (:1339-1525)
// with c = sm_scale log2(e) folded into the register-resident Q (forward, dQ)
// or K (dK/dV).  Delta comes from k_delta_simt (kd_simt.hip).
//
// Why a 16 x 16 product.  With 32 tokens per wave (the 32 x 32 x 2 form,
// which these kernels replaced) a lane holds WD / 2 floats of each register
// row and WD / 2 accumulators per output; at WD = 256 that is more than one
// wave's registers once the compiler's copies are counted, and at WD = 32-128
// its 64-row tiles took twice the LDS of 32-row chunks for no gain.  With 16 tokens per wave a register row is
// WD / 4 floats a lane and a [WD x 16] accumulator WD / 4, so at WD = 256 the
// forward holds ~150 values, dQ ~240 and dK/dV ~310, within one wave per SIMD
// (512 registers).  The 16 x 16 x 4 form runs at the same rate as the 32 x 32
// x 2 one (2048 FLOP in 8 passes against 4096 in 16).
//
// The MFMA.  D[16 x 16] += A[16 x 4] B[4 x 16]: lane l (i = l % 16, g = l / 16)
// supplies A[i][g] and B[g][i], and register r of the result holds D[4 g + r][i].
// Every product keeps the streamed chunk's tokens or head-dim columns on the
// rows of the result and the wave's own 16 tokens on its columns (lane i):
//   forward, dQ:  S^T[key][query] = K Q^T, dP^T = V dO^T: a lane owns one
//                 query; O^T / dQ^T [d][query] += V^T / K^T P^T / dS^T.
//   dK/dV:        S[query][key] = Q K^T, dP = dO V^T: a lane owns one key;
//                 dV^T / dK^T [d][key] += dO^T P / Q^T dS.
// Contraction orders are chosen so that the operands line up without moving
// data between lanes:
//   * over the head dim, k-step 4u + t contracts column 16u + 4g + t on lane
//     group g: a lane reads four k-steps of its A row with one 16-byte LDS read,
//     and the register row is held in that order (reg[4u + t]);
//   * over the chunk's tokens, k-step (kb, r) contracts token 16 kb + 4 g + r
//     on lane group g, which is where register r of score block kb already
//     holds it: the scores are the B operand as they stand;
//   * output block db (of NDB = WD / 16) row 4 g + r is head-dim column
//     NDB (4 g + r) + db, so a lane's A reads for the NDB blocks of one k-step
//     are NDB consecutive floats of one row (NDB / 4 16-byte reads).
//
// Workgroup: 4 waves x 16 tokens = one 64-token member of a 128-token plan
// block (workgroups 2 w and 2 w + 1 take the two members of block w), blocks
// head-major (xcd_remap) and in the plan's longest-first order.  A member
// whose class is EMPTY for a list entry skips it altogether (no copy, no
// product).  The entry's 64 tokens are streamed as two 32-row chunks (32 WD
// fp32 values each: 32 KiB at WD = 256), copied global -> LDS by
// buffer_load ... lds one chunk ahead into two slots.
//
// LDS layout of a chunk row (CPR = WD / 4 chunks of 16 bytes): logical chunk
// c of row r sits at c ^ (r & 15) ^ ((c >> 4) & (CPR / 16 - 1)).  Both read
// patterns are bank-conflict free: (a) 16 lanes read one chunk of 16
// different rows (the r & 15 term spreads them over all 64 banks), (b) 16
// lanes read chunks (NDB / 4) i + j (i = 0..15, fixed j) of one row (the
// (c >> 4) term does, where those chunks span more than 256 bytes).
#include "kd_tile.h"

namespace kd {
namespace {

constexpr int CH = 32;  // rows per streamed chunk

template <int WD>
struct Geo {
  static constexpr int CROWB = WD * 4;        // bytes per chunk row
  static constexpr int CBYTES = CH * CROWB;   // bytes per chunk
  static constexpr int CPR = WD / 4;          // 16-byte chunks per row
  static constexpr int NDB = WD / 16;         // output blocks of 16 rows
  static constexpr int NR = WD / 4;           // floats of a register row per lane
  static constexpr int RPL = 1024 / CROWB;    // rows per wave-wide 1 KiB load
  static constexpr int LPW = CH / RPL / 4;    // such loads per wave and chunk
  static constexpr int HMASK = CPR >= 16 ? CPR / 16 - 1 : 0;  // chunk bits above the low four, folded in
  // workgroups per CU the kernels are built for (1: up to 512 registers a
  // wave; the LDS of two chunk slots of two operands, 4 CBYTES, allows 1, 2,
  // 4, 9 at WD = 256, 128, 64, 32)
  static constexpr int WAVES = WD == 256 ? 1 : WD == 128 ? 2 : WD == 64 ? 3 : 4;
  static_assert(WD == 32 || WD == 64 || WD == 128 || WD == 256, "head dims 32, 64, 128, 256");
  // position of logical 16-byte chunk c in chunk row r (an involution for a
  // fixed r): at WD = 32 a row is 128 bytes, two rows a bank sweep, and 16
  // rows read at one chunk fill the 64 banks once with the row pair's half
  // (r & 1) and the chunk XOR (r >> 1) & 7
  KD_DEV static int pos(int r, int c) {
    if constexpr (WD == 32) return c ^ ((r >> 1) & 7);
    else return c ^ (r & 15) ^ ((c >> 4) & HMASK);
  }
  // byte offset of logical 16-byte chunk c of chunk row r
  KD_DEV static int cat(int r, int c) { return r * CROWB + (pos(r, c) << 4); }
};

KD_DEV f32x4 mma16(float a, float b, const f32x4& c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// This wave's share of the copy of rows r0 .. r0 + 31 of an fp32
// [T, row_bytes] slice into an LDS chunk: wave-wide 16-byte-per-lane loads of
// 1 KiB (RPL rows each), lane l filling chunk position l % CPR of row
// l / CPR of its load, i.e. the logical chunk whose position that is.  Rows
// at or past T read as zeros, and so do the columns from dbytes on (head dim
// 16 on the WD = 32 kernels: their offsets go outside the buffer resource).
template <int WD>
KD_DEV void copy_chunk(const u32x4& rs, uint32_t r0, uint32_t row_bytes, uint32_t lds_chunk, int wave, int lane,
                       uint32_t dbytes) {
  using G = Geo<WD>;
#pragma unroll
  for (int j = 0; j < G::LPW; ++j) {
    const int ld = G::LPW * wave + j;                   // load index within the chunk
    const int rr = ld * G::RPL + lane / G::CPR, p = lane % G::CPR;  // row, position
    const int c = G::pos(rr, p);  // (pos is its own inverse for a fixed row)
    const uint32_t m = uint32_t(__builtin_amdgcn_readfirstlane(int(lds_chunk + uint32_t(ld) * 1024u)));
    dma_b128(rs, col_masked((r0 + uint32_t(rr)) * row_bytes + uint32_t(c) * 16u, uint32_t(c) * 16u, dbytes), m);
  }
}

// this lane's row x[row][.] in k-step order: out[4u + t] = x[row][16u + 4g + t] * scale,
// zero from column dreal on (a row of dreal < WD floats, not read past its end)
template <int WD>
KD_DEV void load_row16(const float* base, int64_t row_stride, int row, bool valid, int g, float scale,
                       float (&out)[Geo<WD>::NR], int dreal) {
  const float* p = base + int64_t(valid ? row : 0) * row_stride + 4 * g;  // row 0 stands in past T
  const float sc = valid ? scale : 0.f;
#pragma unroll
  for (int u = 0; u < WD / 16; ++u) {
    const f32x4 x = 16 * u + 4 * g < dreal ? *reinterpret_cast<const f32x4*>(p + 16 * u) : f32x4{};
#pragma unroll
    for (int t = 0; t < 4; ++t) out[4 * u + t] = x[t] * sc;
  }
}

// Scores of chunk rows 16 kb .. 16 kb + 15 against the lane's register row:
// register r of the result = sum_d chunk[16 kb + 4 g + r][d] reg-row[d].  Both
// blocks at once (two independent chains); each 16-byte read is issued one
// group of four k-steps ahead of its MFMAs.
template <int WD>
KD_DEV void score_pair(const uint8_t* chunk, int i, int g, const float (&reg)[Geo<WD>::NR], f32x4 (&s)[2]) {
  s[0] = s[1] = f32x4{};
  auto rd = [&](int kb, int u) { return *reinterpret_cast<const f32x4*>(chunk + Geo<WD>::cat(16 * kb + i, 4 * u + g)); };
  f32x4 a0 = rd(0, 0), a1 = rd(1, 0);
#pragma unroll
  for (int u = 0; u < WD / 16; ++u) {
    f32x4 n0 = a0, n1 = a1;
    if (u + 1 < WD / 16) {
      n0 = rd(0, u + 1);
      n1 = rd(1, u + 1);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      s[0] = mma16(a0[t], reg[4 * u + t], s[0]);
      s[1] = mma16(a1[t], reg[4 * u + t], s[1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    a0 = n0;
    a1 = n1;
  }
}

// acc[db] (the [d][token] product, NDB blocks) += chunk^T B over the chunk's
// 32 rows, B = the score-shaped registers s (row 16 kb + 4 g + r in register r
// of s[kb]).  For k-step (kb, r) lane (i, g) reads columns NDB i .. NDB i +
// NDB - 1 of chunk row 16 kb + 4 g + r, one float per output block.
template <int WD>
KD_DEV void accumulate16(const uint8_t* chunk, int i, int g, const f32x4 (&s)[2], f32x4 (&acc)[Geo<WD>::NDB]) {
  using G = Geo<WD>;
  if constexpr (G::NDB == 2) {  // WD = 32: two floats (8 bytes) a lane and k-step
    auto rd = [&](int step) {
      const int row = 16 * (step >> 2) + 4 * g + (step & 3);
      return *reinterpret_cast<const f32x2*>(chunk + G::cat(row, i >> 1) + 8 * (i & 1));
    };
    f32x2 a = rd(0);
#pragma unroll
    for (int step = 0; step < 8; ++step) {
      const f32x2 nx = step + 1 < 8 ? rd(step + 1) : a;
      const float b = s[step >> 2][step & 3];
      acc[0] = mma16(a[0], b, acc[0]);
      acc[1] = mma16(a[1], b, acc[1]);
      __builtin_amdgcn_sched_barrier(0);
      a = nx;
    }
    return;
  }
  constexpr int NC = G::NDB >= 4 ? G::NDB / 4 : 1;  // 16-byte reads per k-step
  auto rd = [&](int step, f32x4 (&a)[NC]) {
    const int row = 16 * (step >> 2) + 4 * g + (step & 3);
#pragma unroll
    for (int j = 0; j < NC; ++j) a[j] = *reinterpret_cast<const f32x4*>(chunk + G::cat(row, NC * i + j));
  };
  f32x4 a[NC];
  rd(0, a);
#pragma unroll
  for (int step = 0; step < 8; ++step) {
    f32x4 nx[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) nx[j] = a[j];
    if (step + 1 < 8) rd(step + 1, nx);
    const float b = s[step >> 2][step & 3];
#pragma unroll
    for (int db = 0; db < G::NDB; ++db) acc[db] = mma16(a[db >> 2][db & 3], b, acc[db]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NC; ++j) a[j] = nx[j];
  }
}

// store the [d][token] accumulators of this lane's token to row `out`, times
// scale: register r of block db is column NDB (4 g + r) + db; only the
// columns below dreal (a multiple of NDB) are stored
template <int WD>
KD_DEV void store16(float* out, const f32x4 (&acc)[Geo<WD>::NDB], int g, float scale, int dreal) {
  constexpr int NDB = Geo<WD>::NDB;
  if constexpr (NDB == 2) {  // WD = 32
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (2 * (4 * g + r) < dreal)
        *reinterpret_cast<f32x2*>(out + 2 * (4 * g + r)) = f32x2{acc[0][r] * scale, acc[1][r] * scale};
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < NDB / 4; ++j) {
      const f32x4 x = {acc[4 * j][r] * scale, acc[4 * j + 1][r] * scale, acc[4 * j + 2][r] * scale,
                       acc[4 * j + 3][r] * scale};
      *reinterpret_cast<f32x4*>(out + NDB * (4 * g + r) + 4 * j) = x;
    }
}

// a lane's value combined with those of lanes l ^ 16, l ^ 32, l ^ 48 (the
// four lane groups that hold one token's 16 chunk rows)
KD_DEV float group_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  return xhalf_max(x);
}
KD_DEV float group_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  return xhalf_sum(x);
}

// Work item of this workgroup: head hh, plan item (batch row, block) and member.
struct Item {
  int hh, b, blk, member;
};
KD_DEV Item item_of(const AttnArgs& a, int nblk, const uint32_t* order) {
  const int work = xcd_remap(blockIdx.x, gridDim.x);  // head-major
  const int per_head = 2 * a.B * nblk;
  const int hh = work / per_head, r = work - hh * per_head;
  const int item = int(order[r >> 1]);  // the plan's longest-first order, both members together
  const int b = item / nblk;
  return Item{hh, b, item - b * nblk, r & 1};
}

// index of the first entry at or after e whose class is not EMPTY for member
KD_DEV int next_live(const uint32_t* ent, int e, int n, int member) {
  while (e < n && entry_class(ent[e], member) == TILE_EMPTY) ++e;
  return e;
}

// ------------------------------------------------------------------ forward
template <int WD>
__global__ __launch_bounds__(256, Geo<WD>::WAVES) void k_fwd_f32w(AttnArgs a, const uint32_t* __restrict__ codes,
                                                     const uint32_t* __restrict__ list,
                                                     const int32_t* __restrict__ count, int nT, int nblk,
                                                     const uint32_t* __restrict__ order) {
  using G = Geo<WD>;
  constexpr int NR = G::NR, NDB = G::NDB;
  const uint32_t dbytes = uint32_t(a.D) * 4u;  // a row of a.D <= WD floats (16 on the WD = 32 kernels)
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][G::CBYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][G::CBYTES];
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, i = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Item it = item_of(a, nblk, order);
  const int T = a.T, bh = it.b * a.H + it.hh;
  const int q = it.blk * 128 + it.member * 64 + wave * 16 + i;  // this lane's query
  const bool qvalid = q < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + it.b * a.q_strides[0] + it.hh * a.q_strides[1];
  const float* kg = static_cast<const float*>(a.k) + it.b * a.k_strides[0] + it.hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + it.b * a.v_strides[0] + it.hh * a.v_strides[1];
  const uint32_t krb = uint32_t(a.k_strides[2]) * 4u, vrb = uint32_t(a.v_strides[2]) * 4u;
  const u32x4 rs_k = rsrc_words(kg, uint32_t(T) * krb), rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(it.b) * T, uint32_t(T) * 4u);
  uint32_t qcode = qvalid ? codes[int64_t(it.b) * T + q] : 0u;

  float qr[NR];
  load_row16<WD>(qg, a.q_strides[2], q, qvalid, g, cs, qr, a.D);

  const int lb = it.b * nblk + it.blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  // chunk (entry e, half hf): keys 64 tile + 32 hf .. + 31
  auto copy = [&](int e, int hf, int slot) {
    const uint32_t r0 = entry_tile(ent[e]) * 64u + uint32_t(32 * hf);
    copy_chunk<WD>(rs_k, r0, krb, lds_addr(s_k[slot]), wave, lane, dbytes);
    copy_chunk<WD>(rs_v, r0, vrb, lds_addr(s_v[slot]), wave, lane, dbytes);
    if (wave == 0)
      dma_b32(rs_c, (r0 + uint32_t(lane)) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_kc[slot])))));
  };
  int e = next_live(ent, 0, n, it.member), hf = 0, slot = 0;
  if (e < n) copy(e, 0, 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < NR; ++j) settle(qr[j]);
  settle(qcode);

  f32x4 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x4{};
  float m = -__builtin_inff(), l = 0.f;
  while (e < n) {
    wait_vmem();
    barrier_raw();  // chunk (e, hf) landed for every wave; every wave is done with the other slot
    const uint32_t en = ent[e];
    int ne = e, nh = hf + 1;
    if (nh == 2) {
      nh = 0;
      ne = next_live(ent, e + 1, n, it.member);
    }
    if (ne < n) copy(ne, nh, slot ^ 1);
    f32x4 s[2];
    score_pair<WD>(s_k[slot], i, g, qr, s);
    if (entry_class(en, it.member) == TILE_PARTIAL) {
      const int k0 = int(entry_tile(en)) * 64 + 32 * hf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kc = *reinterpret_cast<const u32x4*>(&s_kc[slot][16 * kb + 4 * g]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s[kb][r] = allow(qcode, kc[r], q, k0 + 16 * kb + 4 * g + r) ? s[kb][r] : -__builtin_inff();
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    const float m_new = fmaxf(m, group_max(mx));
    const float mu = m_new == -__builtin_inff() ? 0.f : m_new;  // rows with nothing allowed yet keep P = 0
    const float alpha = fast_exp2(m - mu);                       // 0 while m is -inf
    m = m_new;
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[kb][r] = fast_exp2(s[kb][r] - mu);
        ls += s[kb][r];
      }
    l = l * alpha + group_sum(ls);
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= alpha;
    accumulate16<WD>(s_v[slot], i, g, s, o);
    e = ne;
    hf = nh;
    slot ^= 1;
  }
  if (!qvalid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  store16<WD>(static_cast<float*>(a.o) + it.b * a.o_strides[0] + it.hh * a.o_strides[1] + int64_t(q) * a.o_strides[2], o,
          g, inv, a.D);
  if (g == 0 && a.lse != nullptr) a.lse[int64_t(bh) * T + q] = l > 0.f ? m + fast_log2(l) : -__builtin_inff();
}

// ----------------------------------------------------------------------- dQ
template <int WD>
__global__ __launch_bounds__(256, Geo<WD>::WAVES) void k_dq_f32w(AttnArgs a, const uint32_t* __restrict__ codes,
                                                    const uint32_t* __restrict__ list,
                                                    const int32_t* __restrict__ count, int nT, int nblk,
                                                    const uint32_t* __restrict__ order) {
  using G = Geo<WD>;
  constexpr int NR = G::NR, NDB = G::NDB;
  const uint32_t dbytes = uint32_t(a.D) * 4u;  // a row of a.D <= WD floats (16 on the WD = 32 kernels)
  __shared__ __attribute__((aligned(1024))) uint8_t s_k[2][G::CBYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_v[2][G::CBYTES];
  __shared__ __attribute__((aligned(256))) uint32_t s_kc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, i = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Item it = item_of(a, nblk, order);
  const int T = a.T, bh = it.b * a.H + it.hh;
  const int q = it.blk * 128 + it.member * 64 + wave * 16 + i;
  const bool qvalid = q < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + it.b * a.q_strides[0] + it.hh * a.q_strides[1];
  const float* dog = static_cast<const float*>(a.dout) + it.b * a.do_strides[0] + it.hh * a.do_strides[1];
  const float* kg = static_cast<const float*>(a.k) + it.b * a.k_strides[0] + it.hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + it.b * a.v_strides[0] + it.hh * a.v_strides[1];
  const uint32_t krb = uint32_t(a.k_strides[2]) * 4u, vrb = uint32_t(a.v_strides[2]) * 4u;
  const u32x4 rs_k = rsrc_words(kg, uint32_t(T) * krb), rs_v = rsrc_words(vg, uint32_t(T) * vrb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(it.b) * T, uint32_t(T) * 4u);
  uint32_t qcode = qvalid ? codes[int64_t(it.b) * T + q] : 0u;
  // P = exp2(S c - LSE); a fully masked row (LSE = -inf) gets P = 0
  const float l0 = qvalid ? a.lse[int64_t(bh) * T + q] : -__builtin_inff();
  float lse = l0 == -__builtin_inff() ? __builtin_inff() : l0;
  float ndelta = qvalid ? a.delta[int64_t(bh) * T + q] : 0.f;  // the workspace holds -Delta

  float qr[NR], dr[NR];
  load_row16<WD>(qg, a.q_strides[2], q, qvalid, g, cs, qr, a.D);
  load_row16<WD>(dog, a.do_strides[2], q, qvalid, g, 1.f, dr, a.D);

  const int lb = it.b * nblk + it.blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  auto copy = [&](int e, int hf, int slot) {
    const uint32_t r0 = entry_tile(ent[e]) * 64u + uint32_t(32 * hf);
    copy_chunk<WD>(rs_k, r0, krb, lds_addr(s_k[slot]), wave, lane, dbytes);
    copy_chunk<WD>(rs_v, r0, vrb, lds_addr(s_v[slot]), wave, lane, dbytes);
    if (wave == 0)
      dma_b32(rs_c, (r0 + uint32_t(lane)) * 4u, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_kc[slot])))));
  };
  int e = next_live(ent, 0, n, it.member), hf = 0, slot = 0;
  if (e < n) copy(e, 0, 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    settle(qr[j]);
    settle(dr[j]);
  }
  settle(qcode);
  settle(lse);
  settle(ndelta);

  f32x4 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = f32x4{};
  while (e < n) {
    wait_vmem();
    barrier_raw();
    const uint32_t en = ent[e];
    int ne = e, nh = hf + 1;
    if (nh == 2) {
      nh = 0;
      ne = next_live(ent, e + 1, n, it.member);
    }
    if (ne < n) copy(ne, nh, slot ^ 1);
    f32x4 s[2], dp[2];
    score_pair<WD>(s_k[slot], i, g, qr, s);
    score_pair<WD>(s_v[slot], i, g, dr, dp);
    if (entry_class(en, it.member) == TILE_PARTIAL) {
      const int k0 = int(entry_tile(en)) * 64 + 32 * hf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kc = *reinterpret_cast<const u32x4*>(&s_kc[slot][16 * kb + 4 * g]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s[kb][r] = allow(qcode, kc[r], q, k0 + 16 * kb + 4 * g + r) ? s[kb][r] : -__builtin_inff();
      }
    }
    // dS^T = P^T (dP^T - Delta), in place of S^T
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[kb][r] = fast_exp2(s[kb][r] - lse) * (dp[kb][r] + ndelta);
    accumulate16<WD>(s_k[slot], i, g, s, dq);
    e = ne;
    hf = nh;
    slot ^= 1;
  }
  if (!qvalid) return;
  store16<WD>(static_cast<float*>(a.dq) + it.b * a.dq_strides[0] + it.hh * a.dq_strides[1] + int64_t(q) * a.dq_strides[2],
          dq, g, a.sm_scale, a.D);
}

// -------------------------------------------------------------------- dK/dV
template <int WD>
__global__ __launch_bounds__(256, Geo<WD>::WAVES) void k_dkdv_f32w(AttnArgs a, const uint32_t* __restrict__ codes,
                                                      const uint32_t* __restrict__ list,
                                                      const int32_t* __restrict__ count, int nT, int nblk,
                                                      const uint32_t* __restrict__ order) {
  using G = Geo<WD>;
  constexpr int NR = G::NR, NDB = G::NDB;
  const uint32_t dbytes = uint32_t(a.D) * 4u;  // a row of a.D <= WD floats (16 on the WD = 32 kernels)
  __shared__ __attribute__((aligned(1024))) uint8_t s_q[2][G::CBYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t s_do[2][G::CBYTES];
  __shared__ __attribute__((aligned(256))) float s_lse[2][64];
  __shared__ __attribute__((aligned(256))) float s_dl[2][64];
  __shared__ __attribute__((aligned(256))) uint32_t s_qc[2][64];
  const int tid = threadIdx.x, lane = tid & 63, i = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Item it = item_of(a, nblk, order);
  const int T = a.T, bh = it.b * a.H + it.hh;
  const int k = it.blk * 128 + it.member * 64 + wave * 16 + i;  // this lane's key
  const bool kvalid = k < T;
  const float cs = a.sm_scale * 1.4426950408889634f;

  const float* qg = static_cast<const float*>(a.q) + it.b * a.q_strides[0] + it.hh * a.q_strides[1];
  const float* dog = static_cast<const float*>(a.dout) + it.b * a.do_strides[0] + it.hh * a.do_strides[1];
  const float* kg = static_cast<const float*>(a.k) + it.b * a.k_strides[0] + it.hh * a.k_strides[1];
  const float* vg = static_cast<const float*>(a.v) + it.b * a.v_strides[0] + it.hh * a.v_strides[1];
  const uint32_t qrb = uint32_t(a.q_strides[2]) * 4u, dorb = uint32_t(a.do_strides[2]) * 4u;
  const u32x4 rs_q = rsrc_words(qg, uint32_t(T) * qrb), rs_do = rsrc_words(dog, uint32_t(T) * dorb);
  const u32x4 rs_c = rsrc_words(codes + int64_t(it.b) * T, uint32_t(T) * 4u);
  const u32x4 rs_l = rsrc_words(a.lse + int64_t(bh) * T, uint32_t(T) * 4u);
  const u32x4 rs_d = rsrc_words(a.delta + int64_t(bh) * T, uint32_t(T) * 4u);  // -Delta
  uint32_t kcode = kvalid ? codes[int64_t(it.b) * T + k] : 0u;

  float kr[NR], vr[NR];
  load_row16<WD>(kg, a.k_strides[2], k, kvalid, g, cs, kr, a.D);
  load_row16<WD>(vg, a.v_strides[2], k, kvalid, g, 1.f, vr, a.D);

  const int lb = it.b * nblk + it.blk;
  const int n = count[lb];
  const uint32_t* ent = list + int64_t(lb) * nT;
  // chunk (entry e, half hf): queries 64 tile + 32 hf .. + 31, with their
  // codes, LSE and -Delta (64 values copied, the first 32 used)
  auto copy = [&](int e, int hf, int slot) {
    const uint32_t r0 = entry_tile(ent[e]) * 64u + uint32_t(32 * hf);
    copy_chunk<WD>(rs_q, r0, qrb, lds_addr(s_q[slot]), wave, lane, dbytes);
    copy_chunk<WD>(rs_do, r0, dorb, lds_addr(s_do[slot]), wave, lane, dbytes);
    const uint32_t off = (r0 + uint32_t(lane)) * 4u;
    if (wave == 0) dma_b32(rs_c, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_qc[slot])))));
    if (wave == 1) dma_b32(rs_l, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_lse[slot])))));
    if (wave == 2) dma_b32(rs_d, off, uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(s_dl[slot])))));
  };
  int e = next_live(ent, 0, n, it.member), hf = 0, slot = 0;
  if (e < n) copy(e, 0, 0);
  wait_vmem();
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    settle(kr[j]);
    settle(vr[j]);
  }
  settle(kcode);

  f32x4 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dk[db] = dv[db] = f32x4{};
  while (e < n) {
    wait_vmem();
    barrier_raw();
    const uint32_t en = ent[e];
    int ne = e, nh = hf + 1;
    if (nh == 2) {
      nh = 0;
      ne = next_live(ent, e + 1, n, it.member);
    }
    if (ne < n) copy(ne, nh, slot ^ 1);
    const int q0 = int(entry_tile(en)) * 64 + 32 * hf;
    const bool full = entry_class(en, it.member) == TILE_FULL;
    f32x4 s[2], dp[2];
    score_pair<WD>(s_q[slot], i, g, kr, s);
    score_pair<WD>(s_do[slot], i, g, vr, dp);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int row = 16 * qb + 4 * g;  // rows row .. row + 3 of the chunk are registers 0 .. 3
      const f32x4 lv = *reinterpret_cast<const f32x4*>(&s_lse[slot][row]);
      const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&s_dl[slot][row]);
      bool ok[4];
      if (full) {
#pragma unroll
        for (int r = 0; r < 4; ++r) ok[r] = lv[r] != -__builtin_inff();
      } else {
        const u32x4 qc = *reinterpret_cast<const u32x4*>(&s_qc[slot][row]);
#pragma unroll
        for (int r = 0; r < 4; ++r) ok[r] = (lv[r] != -__builtin_inff()) & allow(qc[r], kcode, q0 + row + r, k);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ex = fast_exp2(s[qb][r] - lv[r]);
        const float p = ok[r] ? ex : 0.f;
        s[qb][r] = p;
        dp[qb][r] = p * (dp[qb][r] + dv4[r]);  // dS
      }
    }
    accumulate16<WD>(s_do[slot], i, g, s, dv);
    accumulate16<WD>(s_q[slot], i, g, dp, dk);
    e = ne;
    hf = nh;
    slot ^= 1;
  }
  if (!kvalid) return;
  store16<WD>(static_cast<float*>(a.dk) + it.b * a.dk_strides[0] + it.hh * a.dk_strides[1] + int64_t(k) * a.dk_strides[2],
          dk, g, a.sm_scale, a.D);
  store16<WD>(static_cast<float*>(a.dv) + it.b * a.dv_strides[0] + it.hh * a.dv_strides[1] + int64_t(k) * a.dv_strides[2],
          dv, g, 1.f, a.D);
}

template <int WD>
void launch_f32w_d(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(a.B, a.T, a.D);
  const uint32_t* codes = reinterpret_cast<const uint32_t*>(plan + L.codes);
  auto lst = [&](size_t off) { return reinterpret_cast<const uint32_t*>(plan + off); };
  auto cnt = [&](size_t off) { return reinterpret_cast<const int32_t*>(plan + off); };
  const unsigned bh2 = 2u * unsigned(a.B) * unsigned(a.H);  // two member workgroups per block
  if (which == 0)
    hipLaunchKernelGGL(k_fwd_f32w<WD>, dim3(bh2 * unsigned(L.n_fwd_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.fwd_list), cnt(L.fwd_count), L.nT, L.n_fwd_blocks, lst(L.fwd_order));
  else if (which == 2)
    hipLaunchKernelGGL(k_dq_f32w<WD>, dim3(bh2 * unsigned(L.n_dq_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.dq_list), cnt(L.dq_count), L.nT, L.n_dq_blocks, lst(L.dq_order));
  else
    hipLaunchKernelGGL(k_dkdv_f32w<WD>, dim3(bh2 * unsigned(L.n_dkdv_blocks)), dim3(256), 0, st, a, codes,
                       lst(L.dkdv_list), cnt(L.dkdv_count), L.nT, L.n_dkdv_blocks, lst(L.dkdv_order));
}

}  // namespace

int launch_f32mma(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st) {
  switch (a.D) {
    case 16:  // on the WD = 32 kernels: columns 16-31 read as zeros, not stored
    case 32: launch_f32w_d<32>(which, a, plan, st); break;
    case 64: launch_f32w_d<64>(which, a, plan, st); break;
    case 128: launch_f32w_d<128>(which, a, plan, st); break;
    default: launch_f32w_d<256>(which, a, plan, st); break;
  }
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
