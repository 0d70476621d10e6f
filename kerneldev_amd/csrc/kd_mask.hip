// Mask metadata -> per-token codes -> 64x64 tile class map -> work lists.
//
// Replaces the per-element, per-tile re-evaluation of the cocktail-party mask
// in every reference kernel (original_kernel.py:457-517, :1249-1328,
// :1435-1514) with one classification pass whose output all attention
// kernels share:
//   codes   u32 [B, T]            token code (layout in kd_common.h)
//   cls     u8  [B, nT, nT]       0 EMPTY / 1 PARTIAL / 2 FULL per 64x64 tile
//   nnz     i32 [B, nT, nT]       allowed entries per tile
//   lists   u32 [B, nRB, nT]      per row block: (tile << 8) | member classes, ascending
//   counts  i32 [B, nRB]
// The plan stores no per-element masks: the attention kernels build a
// PARTIAL tile's 64-bit row or column masks from the token codes with a few
// wave ballots (query_row_mask / key_col_mask, kd_common.h) and then mask it
// with two VALU ops per score, so the plan grows with B T + B nT^2 bytes
// rather than B nT^2 512.  kd_tile_masks materialises those masks.
#include "kd_internal.h"

namespace kd {

// ---- span-group representative -------------------------------------------
// rep[b][j] = min { t : S_t & sid_t > 0 & sid_t == sid_j } for eligible j
// (S_j & sid_j > 0).  That minimum is always the start of a run of equal
// eligible ids, so one pass lists each row's run starts (and their ids) in
// ascending order, and each eligible token takes the first listed run with
// its id: O(T * runs) instead of O(T^2), exact for any int64 span ids.

KD_DEV int64_t load_sid(const MetaArgs& m, int b, int t) {
  if (m.span_id == nullptr) return 0;
  int64_t off = int64_t(b) * m.span_id_strides[0] + int64_t(t) * m.span_id_strides[1];
  return m.span_id_dtype == KD_I64 ? static_cast<const int64_t*>(m.span_id)[off]
                                   : int64_t(static_cast<const int32_t*>(m.span_id)[off]);
}
KD_DEV bool load_flag(const uint8_t* p, const int64_t* st, int b, int t) {
  return p != nullptr && p[int64_t(b) * st[0] + int64_t(t) * st[1]] != 0;
}
KD_DEV bool eligible(const MetaArgs& m, int b, int t, int64_t* sid) {
  *sid = load_sid(m, b, t);
  return m.span_id != nullptr && load_flag(m.in_span, m.in_span_strides, b, t) && *sid > 0;
}

// One 1024-thread workgroup per batch row; thread i takes a contiguous
// segment, counts its run starts, and a block scan gives each segment its
// first output slot, so the list comes out in ascending order.
__global__ __launch_bounds__(1024) void k_runs(MetaArgs m, uint32_t* runs, int64_t* run_sid, int32_t* run_count) {
  __shared__ int s_warp[16];
  const int b = blockIdx.x, tid = threadIdx.x, T = m.T;
  const int seg = (T + 1023) / 1024, t0 = min(T, tid * seg), t1 = min(T, t0 + seg);
  uint32_t* out = runs + int64_t(b) * T;
  int64_t* out_sid = run_sid + int64_t(b) * T;
  // a run starts at an eligible token whose predecessor is not eligible with the same id
  auto scan = [&](auto&& emit) {
    int64_t prev = 0;
    bool prev_el = t0 > 0 && t0 < T && eligible(m, b, t0 - 1, &prev);
    for (int t = t0; t < t1; ++t) {
      int64_t sid;
      const bool el = eligible(m, b, t, &sid);
      if (el && !(prev_el && prev == sid)) emit(t, sid);
      prev_el = el;
      prev = sid;
    }
  };
  int cnt = 0;
  scan([&](int, int64_t) { ++cnt; });
  const int incl = block_scan(cnt, s_warp);
  int pos = incl - cnt;
  scan([&](int t, int64_t sid) {
    out[pos] = uint32_t(t);
    out_sid[pos] = sid;
    ++pos;
  });
  if (tid == int(blockDim.x) - 1) run_count[b] = incl;
}

// The representative of eligible token t of row b: the first listed run
// with its id (always found: t's own run is listed).
KD_DEV uint32_t run_rep(const MetaArgs& m, const uint32_t* runs, const int64_t* run_sid, const int32_t* run_count,
                        int b, int64_t sid) {
  const int n = run_count[b];
  const int64_t* rs = run_sid + int64_t(b) * m.T;
  int i = 0;
  while (i < n - 1 && rs[i] != sid) ++i;
  return runs[int64_t(b) * m.T + i];
}

// ---- token ids -> metadata (kd_plan_build_tokens) -------------------------
// One workgroup per batch row; thread i scans a contiguous segment of it.
// Segment counts of [SPAN] and [ES] are prefix-summed over the threads and the
// first [CLS] / [MASKQ] are block minima; a second pass then writes, with
// n_span(t), n_es(t) the inclusive counts up to t:
//   collate   in_span = n_span(t) - n_es(t-1) > 0   ([SPAN] .. [ES] inclusive)
//   fallback  in_span = n_span(t) - n_es(t) > 0     ([ES] falls outside)
//   span_id = in_span ? n_span(t) : 0, and -1 at [MASKQ] (collate: the first)
//   is_prefix = t <= first [CLS] (none without a [CLS])
// -- the cumulative-count forms of data_builder.py:603-643 and model.py:209-240.
enum : int64_t { TOK_CLS = 1, TOK_SPAN = 3, TOK_ES = 4, TOK_MASKQ = 5 };

__global__ __launch_bounds__(256) void k_token_meta(kd_token_args a, uint8_t* in_span, int64_t* span_id,
                                                    uint8_t* is_prefix) {
  const int b = blockIdx.x, tid = threadIdx.x, T = a.T;
  const int seg = (T + 255) / 256, t0 = min(T, tid * seg), t1 = min(T, t0 + seg);
  auto tok = [&](int t) -> int64_t {
    const int64_t off = int64_t(b) * a.tokens_strides[0] + int64_t(t) * a.tokens_strides[1];
    return a.tokens_dtype == KD_I64 ? static_cast<const int64_t*>(a.tokens)[off]
                                    : int64_t(static_cast<const int32_t*>(a.tokens)[off]);
  };
  int ns = 0, ne = 0, first_cls = T, first_mq = T;
  for (int t = t0; t < t1; ++t) {
    const int64_t x = tok(t);
    ns += x == TOK_SPAN;
    ne += x == TOK_ES;
    if (x == TOK_CLS && first_cls == T) first_cls = t;
    if (x == TOK_MASKQ && first_mq == T) first_mq = t;
  }
  __shared__ int s_ns[256], s_ne[256], s_cls[256], s_mq[256];
  s_ns[tid] = ns;
  s_ne[tid] = ne;
  s_cls[tid] = first_cls;
  s_mq[tid] = first_mq;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // inclusive scans and minima (Hillis-Steele)
    int a_ns = 0, a_ne = 0, a_c = T, a_m = T;
    if (tid >= off) {
      a_ns = s_ns[tid - off];
      a_ne = s_ne[tid - off];
    }
    a_c = s_cls[tid ^ off];
    a_m = s_mq[tid ^ off];
    __syncthreads();
    s_ns[tid] += a_ns;
    s_ne[tid] += a_ne;
    s_cls[tid] = min(s_cls[tid], a_c);
    s_mq[tid] = min(s_mq[tid], a_m);
    __syncthreads();
  }
  const int cls = s_cls[tid], mq = s_mq[tid];  // block minima (butterfly: every thread holds them)
  int n_span = s_ns[tid] - ns, n_es = s_ne[tid] - ne;  // counts before t0
  const bool spans = a.rule != KD_RULE_TEACHER;
  for (int t = t0; t < t1; ++t) {
    const int64_t x = tok(t);
    const int es_before = n_es;
    n_span += x == TOK_SPAN;
    n_es += x == TOK_ES;
    const bool in = spans && (n_span - (a.rule == KD_RULE_COLLATE ? es_before : n_es)) > 0;
    int64_t sid = in ? n_span : 0;
    if (spans && x == TOK_MASKQ && (a.rule == KD_RULE_FALLBACK || t == mq)) sid = -1;
    const int64_t o = int64_t(b) * T + t;
    in_span[o] = in ? 1 : 0;
    span_id[o] = sid;
    is_prefix[o] = (cls < T && t <= cls) ? 1 : 0;
  }
}

// ---- token codes -------------------------------------------------------
// runs / run_sid / run_count: the run-start lists of k_runs (formula mode
// with span ids); rep receives each eligible token's representative.
__global__ void k_codes(MetaArgs m, const uint32_t* runs, const int64_t* run_sid, const int32_t* run_count,
                        uint32_t* rep, uint32_t* codes) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= int64_t(m.B) * m.T) return;
  const int b = int(idx / m.T), t = int(idx % m.T);
  int seq_len = m.T;
  if (m.lens != nullptr) seq_len = min(m.lens[int64_t(b) * m.lens_stride], m.T);
  uint32_t code = 0;
  if (t < seq_len) {
    if (m.mode == KD_MODE_CAUSAL) {
      code = FLAG_C;  // every token context: C & C & i >= j  (:512-513)
    } else if (m.mode == KD_MODE_ALL) {
      code = FLAG_P | (FLAG_P << 4);  // P sees P: every pair (:514-515)
    } else {
      const bool P = load_flag(m.is_prefix, m.is_prefix_strides, b, t);
      const bool S = load_flag(m.in_span, m.in_span_strides, b, t);
      const int64_t sid = load_sid(m, b, t);
      const bool M = m.span_id != nullptr && sid == -1;
      const bool C = !S && !P && !M;
      uint32_t acc = 0;
      if (P || C) acc |= FLAG_P;          // prefix_to_prefix, context_to_prefix
      if (S) acc |= FLAG_C;               // span_to_context
      if (M) acc |= FLAG_S | FLAG_P;      // maskq_to_spans, maskq_to_cls
      code = (P ? FLAG_P : 0u) | (S ? FLAG_S : 0u) | (M ? FLAG_M : 0u) | (C ? FLAG_C : 0u) | (acc << 4);
      if (m.span_id != nullptr && S && sid > 0) {  // same_span: eligible, so k_runs listed its run
        const uint32_t r = run_rep(m, runs, run_sid, run_count, b, sid);
        rep[idx] = r;
        code |= (r + 1u) << 8;
      }
    }
  }
  codes[idx] = code;
}

// ---- 64x64 tile classifier ---------------------------------------------
// One wave per tile.  The row mask of query lane i over the tile's 64 keys is
// built from wave-wide ballots instead of 64 per-key tests: with F_j the key
// flags and A_i the query's allowed flags, A_i & F_j != 0 selects the ballot
// of keys carrying each flag of A_i; context queries add context keys at
// j <= i (all of them below the diagonal, none above); and for the same-span
// term the wave walks the distinct span representatives among the tile's keys
// (usually one to three), one ballot each: query_row_mask, the function the
// forward and dQ kernels use for PARTIAL tiles.  That is the rule of allow(),
// term for term.
__global__ __launch_bounds__(256) void k_tilemap(const uint32_t* codes, int T, int nT, uint8_t* cls,
                                                 int32_t* nnz) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qt = blockIdx.y, b = blockIdx.z;
  const int kt0 = blockIdx.x * 4;
  __shared__ uint32_t s_k[256];
  {
    const int j = kt0 * 64 + threadIdx.x;
    s_k[threadIdx.x] = (j < T) ? codes[int64_t(b) * T + j] : 0u;
  }
  __syncthreads();
  const int kt = kt0 + wave;
  if (kt >= nT) return;
  const int i = qt * 64 + lane;
  const uint32_t qc = (i < T) ? codes[int64_t(b) * T + i] : 0u;
  const uint32_t kc = s_k[wave * 64 + lane];  // key j = 64 kt + lane (code 0 past T: allows nothing)
  const uint64_t row = query_row_mask(qc, i, kc, kt * 64);
  int cnt = __builtin_popcountll(row);
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
  const int64_t o = (int64_t(b) * nT + qt) * nT + kt;
  const uint8_t k = cnt == 0 ? TILE_EMPTY : (cnt == 64 * 64 ? TILE_FULL : TILE_PARTIAL);
  if (lane == 0) {
    cls[o] = k;
    if (nnz != nullptr) nnz[o] = cnt;
  }
}

// ---- tile masks (inspection) -----------------------------------------------
// Every tile's 64 row masks and 64 column masks, from the same functions the
// attention kernels use for PARTIAL tiles.  One wave per tile: lane r is row
// r for query_row_mask and key r for key_col_mask.
__global__ __launch_bounds__(256) void k_tile_masks(const uint32_t* codes, int T, int nT, uint64_t* rows,
                                                    uint64_t* cols) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qt = blockIdx.y, b = blockIdx.z, kt = blockIdx.x * 4 + wave;
  if (kt >= nT) return;  // wave-uniform
  const uint32_t* cb = codes + int64_t(b) * T;
  const int i = qt * 64 + lane, j = kt * 64 + lane;
  const uint32_t qc = i < T ? cb[i] : 0u, kc = j < T ? cb[j] : 0u;
  const int64_t o = ((int64_t(b) * nT + qt) * nT + kt) * 64 + lane;
  rows[o] = query_row_mask(qc, i, kc, kt * 64);
  cols[o] = key_col_mask(kc, j, qc, qt * 64);
}

// ---- per-row-block work lists ------------------------------------------
// One wave per row block: lanes test 64 columns at a time and compact the
// non-empty ones in ascending order with a ballot + prefix popcount; the
// tail of the list is zero-filled.  All three lists build in one launch
// (blockIdx.y picks the list).
struct ListSpec {
  uint32_t* entries;
  int32_t* counts;
  int group, by_key, nrb;
};
struct ListSpecs {
  ListSpec l[3];
};

__global__ __launch_bounds__(64) void k_lists(const uint8_t* __restrict__ cls, int B, int nT, ListSpecs specs) {
  const ListSpec sp = specs.l[blockIdx.y];
  const int idx = blockIdx.x;  // b * nrb + rb
  if (idx >= B * sp.nrb) return;
  const int b = idx / sp.nrb, rb = idx % sp.nrb, lane = threadIdx.x;
  const uint8_t* base = cls + int64_t(b) * nT * nT;
  uint32_t* out = sp.entries + int64_t(idx) * nT;
  int n = 0;
  for (int c0 = 0; c0 < nT; c0 += 64) {
    const int c = c0 + lane;
    bool any_ne = false;
    uint32_t classes = 0;
    if (c < nT) {
      for (int r = 0; r < sp.group; ++r) {
        const int row = rb * sp.group + r;
        uint8_t k = TILE_EMPTY;
        if (row < nT) k = sp.by_key ? base[int64_t(c) * nT + row] : base[int64_t(row) * nT + c];
        any_ne |= (k != TILE_EMPTY);
        classes |= uint32_t(k) << (2 * r);
      }
    }
    const uint64_t m = __builtin_amdgcn_ballot_w64(any_ne);
    const int pos = n + __builtin_popcountll(m & ((uint64_t(1) << lane) - 1));
    if (any_ne) out[pos] = (uint32_t(c) << 8) | classes;
    n += __builtin_popcountll(m);
  }
  for (int c = n + lane; c < nT; c += 64) out[c] = 0;
  if (lane == 0) sp.counts[idx] = n;
}

// ---- work order ----------------------------------------------------------
// Forward and dQ lists: the B n items (b, block) = b n + block sorted by descending list
// length, equal lengths in ascending item order: item i goes to position
// #{j : c_j > c_i or (c_j == c_i and j < i)}.  The attention kernels take
// each head's blocks in this order, so the longest ones start first and the
// short ones fill the end of every XCD's range (longest-first list
// scheduling), instead of a fixed block order whose longest blocks may come
// last.
struct OrderSpecs {
  const int32_t* counts[2];
  uint32_t* order[2];
  int n[2];
};

__global__ __launch_bounds__(256) void k_order(OrderSpecs specs) {
  const int y = blockIdx.y, n = specs.n[y];
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t* c = specs.counts[y];
  const int ci = c[i];
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const int cj = c[j];
    rank += (cj > ci || (cj == ci && j < i)) ? 1 : 0;
  }
  specs.order[y][rank] = uint32_t(i);
}

// ---- dense mask output (return_attention_mask) -------------------------
__global__ void k_mask_dense(const uint32_t* codes, int B, int H, int T, uint8_t* out, int64_t sb,
                             int64_t sh, int64_t sq, int64_t sk) {
  const int64_t n = int64_t(B) * H * T * T;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < n;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int j = int(idx % T);
    const int i = int((idx / T) % T);
    const int h = int((idx / (int64_t(T) * T)) % H);
    const int b = int(idx / (int64_t(T) * T * H));
    const bool a = allow(codes[int64_t(b) * T + i], codes[int64_t(b) * T + j], i, j);
    out[b * sb + h * sh + i * sq + j * sk] = a ? 1 : 0;
  }
}

// ---- host launchers ----------------------------------------------------
PlanLayout plan_layout(int B, int T, int D) {
  PlanLayout L{};
  const int nT = (T + 63) / 64;
  L.nT = nT;
  L.fwd_group = fwd_rows_per_block(D) / 64;
  L.dq_group = dq_rows_per_block(D) / 64;
  L.dkdv_group = dkdv_keys_per_block(D) / 64;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~size_t(255);
    return o;
  };
  const size_t BT = size_t(B) * T, BTT = size_t(B) * nT * nT;
  L.codes = take(BT * 4);
  L.rep = take(BT * 4);
  L.runs = take(BT * 4);
  L.run_sid = take(BT * 8);
  L.run_count = take(size_t(B) * 4);
  L.tok_in_span = take(BT);
  L.tok_span_id = take(BT * 8);
  L.tok_prefix = take(BT);
  L.cls = take(BTT);
  L.nnz = take(BTT * 4);
  const int nf = (nT + L.fwd_group - 1) / L.fwd_group;
  const int nq = (nT + L.dq_group - 1) / L.dq_group;
  const int nk = (nT + L.dkdv_group - 1) / L.dkdv_group;
  L.n_fwd_blocks = nf;
  L.n_dq_blocks = nq;
  L.n_dkdv_blocks = nk;
  L.fwd_list = take(size_t(B) * nf * nT * 4);
  L.fwd_count = take(size_t(B) * nf * 4);
  L.dq_list = take(size_t(B) * nq * nT * 4);
  L.dq_count = take(size_t(B) * nq * 4);
  L.dkdv_list = take(size_t(B) * nk * nT * 4);
  L.dkdv_count = take(size_t(B) * nk * 4);
  L.fwd_order = take(size_t(B) * nf * 4);
  L.dq_order = take(size_t(B) * nq * 4);
  L.total = off;
  return L;
}

int launch_plan(const MetaArgs& m, uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(m.B, m.T, m.D);
  uint32_t* codes = reinterpret_cast<uint32_t*>(plan + L.codes);
  uint32_t* rep = reinterpret_cast<uint32_t*>(plan + L.rep);
  uint8_t* cls = plan + L.cls;
  int32_t* nnz = reinterpret_cast<int32_t*>(plan + L.nnz);
  const int64_t BT = int64_t(m.B) * m.T;
  uint32_t* runs = reinterpret_cast<uint32_t*>(plan + L.runs);
  int64_t* run_sid = reinterpret_cast<int64_t*>(plan + L.run_sid);
  int32_t* run_count = reinterpret_cast<int32_t*>(plan + L.run_count);
  // (k_codes reads the run lists only for eligible tokens, which exist only in this mode)
  if (m.mode == KD_MODE_FORMULA && m.span_id != nullptr && m.in_span != nullptr)
    hipLaunchKernelGGL(k_runs, dim3(unsigned(m.B)), dim3(1024), 0, st, m, runs, run_sid, run_count);
  hipLaunchKernelGGL(k_codes, dim3(unsigned((BT + 255) / 256)), dim3(256), 0, st, m, runs, run_sid, run_count, rep,
                     codes);
  hipLaunchKernelGGL(k_tilemap, dim3((L.nT + 3) / 4, L.nT, m.B), dim3(256), 0, st, codes, m.T, L.nT, cls, nnz);
  ListSpecs specs;
  specs.l[0] = {reinterpret_cast<uint32_t*>(plan + L.fwd_list), reinterpret_cast<int32_t*>(plan + L.fwd_count),
                L.fwd_group, 0, L.n_fwd_blocks};
  specs.l[1] = {reinterpret_cast<uint32_t*>(plan + L.dq_list), reinterpret_cast<int32_t*>(plan + L.dq_count),
                L.dq_group, 0, L.n_dq_blocks};
  specs.l[2] = {reinterpret_cast<uint32_t*>(plan + L.dkdv_list), reinterpret_cast<int32_t*>(plan + L.dkdv_count),
                L.dkdv_group, 1, L.n_dkdv_blocks};
  const int max_rb = std::max(L.n_fwd_blocks, std::max(L.n_dq_blocks, L.n_dkdv_blocks));
  hipLaunchKernelGGL(k_lists, dim3(unsigned(m.B * max_rb), 3), dim3(64), 0, st, cls, m.B, L.nT, specs);
  OrderSpecs os;
  uint32_t* const ords[2] = {reinterpret_cast<uint32_t*>(plan + L.fwd_order), reinterpret_cast<uint32_t*>(plan + L.dq_order)};
  for (int y = 0; y < 2; ++y) {
    os.counts[y] = specs.l[y].counts;
    os.order[y] = ords[y];
    os.n[y] = m.B * specs.l[y].nrb;
  }
  hipLaunchKernelGGL(k_order, dim3(unsigned((m.B * std::max(L.n_fwd_blocks, L.n_dq_blocks) + 255) / 256), 2), dim3(256),
                     0, st, os);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

int launch_plan_tokens(const kd_token_args& t, uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(t.B, t.T, t.D);
  MetaArgs m{};
  m.in_span = plan + L.tok_in_span;
  m.in_span_strides[0] = t.T;
  m.in_span_strides[1] = 1;
  m.span_id = plan + L.tok_span_id;
  m.span_id_strides[0] = t.T;
  m.span_id_strides[1] = 1;
  m.span_id_dtype = KD_I64;
  m.is_prefix = plan + L.tok_prefix;
  m.is_prefix_strides[0] = t.T;
  m.is_prefix_strides[1] = 1;
  m.mode = KD_MODE_FORMULA;
  m.lens = t.lens;
  m.lens_stride = t.lens_stride;
  m.B = t.B;
  m.T = t.T;
  m.D = t.D;
  hipLaunchKernelGGL(k_token_meta, dim3(unsigned(t.B)), dim3(256), 0, st, t, plan + L.tok_in_span,
                     reinterpret_cast<int64_t*>(plan + L.tok_span_id), plan + L.tok_prefix);
  if (hipGetLastError() != hipSuccess) return KD_ERR_LAUNCH;
  return launch_plan(m, plan, st);
}

int launch_tile_masks(const uint8_t* plan, int B, int T, int D, uint64_t* rows, uint64_t* cols, hipStream_t st) {
  const PlanLayout L = plan_layout(B, T, D);
  hipLaunchKernelGGL(k_tile_masks, dim3((L.nT + 3) / 4, L.nT, B), dim3(256), 0, st,
                     reinterpret_cast<const uint32_t*>(plan + L.codes), T, L.nT, rows, cols);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

int launch_mask_dense(const uint32_t* codes, int B, int H, int T, uint8_t* out, const int64_t* s,
                      hipStream_t st) {
  const int64_t n = int64_t(B) * H * T * T;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(k_mask_dense, dim3(unsigned(blocks)), dim3(256), 0, st, codes, B, H, T, out, s[0], s[1],
                     s[2], s[3]);
  return hipGetLastError() == hipSuccess ? KD_OK : KD_ERR_LAUNCH;
}

}  // namespace kd
