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
// its id.  When the ids increase strictly from run to run (checked per row)
// that is the token's own run; otherwise a linear search of the list finds
// it: O(T * runs) at worst instead of O(T^2), exact for any int64 span ids.

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

// The representative of eligible token t of row b: the first listed run
// with its id (always found: t's own run is listed).
KD_DEV uint32_t run_rep(const MetaArgs& m, const uint32_t* runs, const int64_t* run_sid, int n, int b, int64_t sid) {
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

// ---- token codes (first of the plan's three launches) --------------------
// The code of a token (layout in kd_common.h) from its prefix / span / [MASKQ]
// flags, with representative r when has_rep (an eligible token in formula
// mode with span ids).
KD_DEV uint32_t token_code(int mode, bool P, bool S, bool M, bool has_rep, uint32_t r) {
  if (mode == KD_MODE_CAUSAL) return FLAG_C;               // every token context: C & C & i >= j  (:512-513)
  if (mode == KD_MODE_ALL) return FLAG_P | (FLAG_P << 4);  // P sees P: every pair (:514-515)
  const bool C = !S && !P && !M;
  uint32_t acc = 0;
  if (P || C) acc |= FLAG_P;      // prefix_to_prefix, context_to_prefix
  if (S) acc |= FLAG_C;           // span_to_context
  if (M) acc |= FLAG_S | FLAG_P;  // maskq_to_spans, maskq_to_cls
  uint32_t code = (P ? FLAG_P : 0u) | (S ? FLAG_S : 0u) | (M ? FLAG_M : 0u) | (C ? FLAG_C : 0u) | (acc << 4);
  if (has_rep) code |= (r + 1u) << 8;  // same_span
  return code;
}

constexpr int CODE_SEG = 8;  // most tokens per thread and round (span ids)

// Grid (chunks, B) of 1024 threads.  Without span ids each workgroup codes a
// chunk of row b.  With span ids (formula mode) one workgroup takes the row
// whole, in rounds of 1024 seg tokens (seg = T / 1024 rounded up, at most
// CODE_SEG): thread i loads the metadata of its seg consecutive tokens (and
// of the token before) at once, marks the
// run starts (eligible tokens whose predecessor is not eligible with the same
// id), and a block scan gives its first slot in the row's ascending list of
// run starts (runs, run_sid).  It then codes its tokens, taking as each
// eligible token's representative its own run's start -- the start of the run
// before its first slot for a run that began earlier.  That is the first run
// with the token's id whenever the ids increase strictly from run to run
// (each id has one run), the layout of the token-derived metadata and of the
// collate builders; the workgroup checks that over the finished list and
// otherwise recodes the eligible tokens with the first listed run with their
// id (run_rep).  The workgroups also zero the forward and dK/dV list lengths,
// which the tile classifier accumulates.
__global__ __launch_bounds__(1024) void k_codes_rows(MetaArgs m, uint32_t* runs, int64_t* run_sid, int32_t* run_count,
                                                     uint32_t* rep, uint32_t* codes, int32_t* fwd_n, int n_fwd,
                                                     int32_t* dkdv_n, int n_dkdv) {
  __shared__ int s_warp[16];
  __shared__ int s_n, s_dup;
  const int b = blockIdx.y, tid = threadIdx.x, T = m.T;
  const bool spans = m.mode == KD_MODE_FORMULA && m.span_id != nullptr && m.in_span != nullptr;
  {
    const int gid = (blockIdx.y * gridDim.x + blockIdx.x) * 1024 + tid, nth = gridDim.x * gridDim.y * 1024;
    for (int i = gid; i < n_fwd; i += nth) fwd_n[i] = 0;
    for (int i = gid; i < n_dkdv; i += nth) dkdv_n[i] = 0;
  }
  int seq_len = T;
  if (m.lens != nullptr) seq_len = min(m.lens[int64_t(b) * m.lens_stride], T);
  if (!spans) {
    const int per = (T + gridDim.x - 1) / gridDim.x;
    const int c0 = blockIdx.x * per, c1 = min(T, c0 + per);
    for (int t = c0 + tid; t < c1; t += 1024) {
      uint32_t code = 0;
      if (t < seq_len) {
        const bool P = load_flag(m.is_prefix, m.is_prefix_strides, b, t);
        const bool S = load_flag(m.in_span, m.in_span_strides, b, t);
        const bool M = m.span_id != nullptr && load_sid(m, b, t) == -1;
        code = token_code(m.mode, P, S, M, false, 0u);
      }
      codes[int64_t(b) * T + t] = code;
    }
    return;
  }
  // (gridDim.x == 1 in this mode)
  if (tid == 0) s_dup = 0;
  uint32_t* out = runs + int64_t(b) * T;
  int64_t* out_sid = run_sid + int64_t(b) * T;
  int n_before = 0;  // runs listed in earlier rounds
  const int seg = min(CODE_SEG, (T + 1023) / 1024);
  for (int base = 0; base < T; base += 1024 * seg) {
    const int t0 = base + tid * seg;
    int64_t prev = 0;
    const bool prev_el = t0 > 0 && t0 < T && eligible(m, b, t0 - 1, &prev);
    bool P[CODE_SEG], S[CODE_SEG], el[CODE_SEG], st[CODE_SEG];
    int64_t sid[CODE_SEG];
#pragma unroll
    for (int k = 0; k < CODE_SEG; ++k) {
      const int t = t0 + k;
      const bool in = k < seg && t < T;
      sid[k] = in ? load_sid(m, b, t) : 0;
      S[k] = in && load_flag(m.in_span, m.in_span_strides, b, t);
      P[k] = in && load_flag(m.is_prefix, m.is_prefix_strides, b, t);
      el[k] = S[k] && sid[k] > 0;
    }
    int cnt = 0;
    {
      bool pe = prev_el;
      int64_t ps = prev;
#pragma unroll
      for (int k = 0; k < CODE_SEG; ++k) {
        st[k] = el[k] && !(pe && ps == sid[k]);
        cnt += st[k];
        pe = el[k];
        ps = sid[k];
      }
    }
    const int incl = block_scan(cnt, s_warp);
    const int first = n_before + incl - cnt;
    int pos = first;
#pragma unroll
    for (int k = 0; k < CODE_SEG; ++k)
      if (st[k]) {
        out[pos] = uint32_t(t0 + k);
        out_sid[pos] = sid[k];
        ++pos;
      }
    if (tid == 1023) s_n = n_before + incl;
    __syncthreads();
    // the run token t0 - 1 belongs to (if eligible): the last one listed before this thread's first slot
    uint32_t start = (prev_el && first > 0) ? out[first - 1] : 0u;
#pragma unroll
    for (int k = 0; k < CODE_SEG; ++k) {
      const int t = t0 + k;
      if (k >= seg || t >= T) break;
      if (st[k]) start = uint32_t(t);
      const int64_t idx = int64_t(b) * T + t;
      uint32_t code = 0;
      if (t < seq_len) {
        if (el[k]) rep[idx] = start;
        code = token_code(m.mode, P[k], S[k], sid[k] == -1, el[k], start);
      }
      codes[idx] = code;
    }
    n_before = s_n;  // (s_n is next written after the next round's block scan barriers)
  }
  if (tid == 0) run_count[b] = n_before;
  for (int i = tid; i + 1 < n_before; i += 1024)
    if (out_sid[i] >= out_sid[i + 1]) s_dup = 1;
  __syncthreads();
  if (s_dup == 0) return;  // workgroup-uniform
  for (int t = tid; t < seq_len; t += 1024) {
    int64_t sid;
    if (!eligible(m, b, t, &sid)) continue;
    const int64_t idx = int64_t(b) * T + t;
    const uint32_t r = run_rep(m, runs, run_sid, n_before, b, sid);
    rep[idx] = r;
    codes[idx] = (codes[idx] & 0xFFu) | ((r + 1u) << 8);
  }
}

// ---- 64x64 tile classifier (second launch) ------------------------------
// Four waves per workgroup, on the two q-tiles of row block blockIdx.y and
// 2 kpw consecutive k-tiles: wave w takes q-tile 2 rb + (w & 1) against the
// kpw k-tiles of half (w >> 1), one after another (kpw > 1 on large plans,
// where the grid fills the chip anyway and each wave's loads and barrier then
// serve more tiles).  The row mask of query lane i
// over a tile's 64 keys is built from wave-wide ballots instead of 64
// per-key tests: with F_j the key flags and A_i the query's allowed flags,
// A_i & F_j != 0 selects the ballot of keys carrying each flag of A_i;
// context queries add context keys at j <= i (all of them below the diagonal,
// none above); and for the same-span term the wave walks the distinct span
// representatives among the tile's keys (usually one to three), one ballot
// each: query_row_mask, the function the forward and dQ kernels use for
// PARTIAL tiles.  That is the rule of allow(), term for term.  The workgroup
// then adds its k-tiles with a non-empty tile in the row block to that row
// block's forward list length, and for each of its key blocks (k-tiles
// 2 kb, 2 kb + 1) its q-tiles with a non-empty tile there to that key block's
// dK/dV list length (both zeroed by the first launch).
constexpr int TM_KPW = 4;  // most k-tiles per wave

__global__ __launch_bounds__(256) void k_tilemap(const uint32_t* codes, int T, int nT, int kpw, int nqb, uint8_t* cls,
                                                 int32_t* nnz, int32_t* fwd_n, int32_t* dkdv_n, int nkb) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.z, half = wave >> 1;
  const int kt0 = blockIdx.x * 2 * kpw;
  __shared__ uint32_t s_k[2 * TM_KPW * 64];
  __shared__ uint32_t s_ne[2];  // bit i: k-tile kt0 + i has a non-empty tile, per q-tile
  for (int x = threadIdx.x; x < 2 * kpw * 64; x += 256) {
    const int j = kt0 * 64 + x;
    s_k[x] = (j < T) ? codes[int64_t(b) * T + j] : 0u;
  }
  // row blocks blockIdx.y, + gridDim.y, ... (the grid's y extent is capped at 65535)
  for (int rb = blockIdx.y; rb < nqb; rb += gridDim.y) {
    if (threadIdx.x < 2) s_ne[threadIdx.x] = 0u;
    __syncthreads();  // s_k landed (first pass), s_ne cleared
    const int qt = rb * 2 + (wave & 1);
    const int i = qt * 64 + lane;
    const uint32_t qc = (qt < nT && i < T) ? codes[int64_t(b) * T + i] : 0u;
    uint32_t ne = 0;
    if (qt < nT) {  // wave-uniform
      for (int x = half * kpw; x < (half + 1) * kpw; ++x) {
        const int kt = kt0 + x;
        if (kt >= nT) break;
        const uint32_t kc = s_k[x * 64 + lane];  // key j = 64 kt + lane (code 0 past T: allows nothing)
        const uint64_t row = query_row_mask(qc, i, kc, kt * 64);
        int cnt = __builtin_popcountll(row);
        for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
        const int64_t o = (int64_t(b) * nT + qt) * nT + kt;
        if (lane == 0) {
          cls[o] = cnt == 0 ? TILE_EMPTY : (cnt == 64 * 64 ? TILE_FULL : TILE_PARTIAL);
          if (nnz != nullptr) nnz[o] = cnt;
        }
        if (cnt != 0) ne |= 1u << x;
      }
    }
    if (lane == 0 && ne != 0u) atomicOr(&s_ne[wave & 1], ne);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int add = __builtin_popcount(s_ne[0] | s_ne[1]);
      if (add != 0) atomicAdd(fwd_n + int64_t(b) * nqb + rb, add);
    } else if (int(threadIdx.x) <= kpw) {  // key block j = threadIdx.x - 1 of this workgroup
      const int j = int(threadIdx.x) - 1, kb = int(blockIdx.x) * kpw + j;
      const int add = int(((s_ne[0] >> (2 * j)) & 3u) != 0u) + int(((s_ne[1] >> (2 * j)) & 3u) != 0u);
      if (kb < nkb && add != 0) atomicAdd(dkdv_n + int64_t(b) * nkb + kb, add);
    }
    __syncthreads();  // every read of s_ne done before the next pass clears it
  }
}

// ---- work lists and work orders (third launch) ----------------------------
// One workgroup per list: the B nqb row blocks of the forward / dQ lists (two
// q-tiles against every k-tile; the two lists are the same), then the B nkb
// key blocks of the dK/dV list (two k-tiles against every q-tile).  Wave 0
// compacts the block's non-empty entries in ascending order with a ballot and
// a prefix popcount, and zero-fills the tail.  A work order ranks a list's
// B n items b n + block by descending list length, equal lengths in ascending
// item order (item i goes to position #{j : c_j > c_i or (c_j == c_i and
// j < i)}); the kernels that use one take each head's blocks in this order,
// so the longest start first and the short ones fill the end of every XCD's
// range (longest-first list scheduling).  The list lengths arrive complete
// from the classifier, so each workgroup ranks its own item and no workgroup
// waits for another.
struct ListOut {
  uint32_t *fwd, *dq, *dkdv;       // entries, [B nb nT]
  int32_t *fwd_n, *dq_n, *dkdv_n;  // counts, [B nb]
  uint32_t *fwd_order, *dq_order;  // [B nqb]
  uint32_t* dkdv_order;            // [B nkb]
  int nqb, nkb;                    // row blocks (forward and dQ), key blocks (dK/dV)
};

// entry class bits of block rb (tiles 2 rb, 2 rb + 1) against tile c of the
// other axis (by_key: the block's tiles are key tiles, a column of the map)
KD_DEV uint32_t block_classes(const uint8_t* cls_b, int nT, int rb, int c, bool by_key) {
  uint32_t classes = 0;
  for (int r = 0; r < 2; ++r) {
    const int t = rb * 2 + r;
    if (t < nT) classes |= uint32_t(by_key ? cls_b[int64_t(c) * nT + t] : cls_b[int64_t(t) * nT + c]) << (2 * r);
  }
  return classes;
}

__global__ __launch_bounds__(256) void k_lists(const uint8_t* __restrict__ cls, int nT, ListOut lo) {
  __shared__ int s_cnt[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int B = int(gridDim.y), b = blockIdx.y;
  const bool rows = int(blockIdx.x) < lo.nqb;  // a row block of the forward / dQ lists, else a key block
  const int blk = rows ? int(blockIdx.x) : int(blockIdx.x) - lo.nqb;
  const int item = b * (rows ? lo.nqb : lo.nkb) + blk;
  if (wave == 0) {
    const uint8_t* cls_b = cls + int64_t(b) * nT * nT;
    uint32_t* out = (rows ? lo.fwd : lo.dkdv) + int64_t(item) * nT;
    uint32_t* out2 = rows ? lo.dq + int64_t(item) * nT : nullptr;
    int n = 0;
    for (int c0 = 0; c0 < nT; c0 += 64) {
      const int c = c0 + lane;
      const uint32_t classes = c < nT ? block_classes(cls_b, nT, blk, c, !rows) : 0u;
      const bool any_ne = classes != 0u;
      const uint64_t msk = __builtin_amdgcn_ballot_w64(any_ne);
      const int pos = n + __builtin_popcountll(msk & ((uint64_t(1) << lane) - 1));
      if (any_ne) {
        out[pos] = (uint32_t(c) << 8) | classes;
        if (rows) out2[pos] = (uint32_t(c) << 8) | classes;
      }
      n += __builtin_popcountll(msk);
    }
    for (int c = n + lane; c < nT; c += 64) {
      out[c] = 0;
      if (rows) out2[c] = 0;
    }
    if (lane == 0 && rows) lo.dq_n[item] = n;  // (fwd_n, dkdv_n: the classifier's sums, the same n)
  }
  // this item's rank: the items before it in the order
  const int32_t* len = rows ? lo.fwd_n : lo.dkdv_n;
  const int ci = len[item], n_items = B * (rows ? lo.nqb : lo.nkb);
  int before = 0;
  for (int j = tid; j < n_items; j += 256) {
    const int cj = len[j];
    before += (cj > ci || (cj == ci && j < item)) ? 1 : 0;
  }
  for (int off = 32; off > 0; off >>= 1) before += __shfl_xor(before, off);
  if (lane == 0) s_cnt[wave] = before;
  __syncthreads();
  if (tid == 0) {
    const int rank = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    if (rows) {
      lo.fwd_order[rank] = uint32_t(item);
      lo.dq_order[rank] = uint32_t(item);
    } else {
      lo.dkdv_order[rank] = uint32_t(item);
    }
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
  L.dkdv_order = take(size_t(B) * nk * 4);
  L.total = off;
  return L;
}

int launch_plan(const MetaArgs& m, uint8_t* plan, hipStream_t st) {
  const PlanLayout L = plan_layout(m.B, m.T, m.D);
  uint32_t* codes = reinterpret_cast<uint32_t*>(plan + L.codes);
  uint32_t* rep = reinterpret_cast<uint32_t*>(plan + L.rep);
  uint8_t* cls = plan + L.cls;
  int32_t* nnz = reinterpret_cast<int32_t*>(plan + L.nnz);
  uint32_t* runs = reinterpret_cast<uint32_t*>(plan + L.runs);
  int64_t* run_sid = reinterpret_cast<int64_t*>(plan + L.run_sid);
  int32_t* run_count = reinterpret_cast<int32_t*>(plan + L.run_count);
  // k_tilemap and k_lists build lists of blocks of two 64-row tiles
  if (L.fwd_group != 2 || L.dq_group != 2 || L.dkdv_group != 2) return KD_ERR_UNSUPPORTED;
  // formula mode with span ids: one workgroup per row (it lists the row's
  // runs before coding its tokens); otherwise chunks of 8 tokens a thread
  const bool spans = m.mode == KD_MODE_FORMULA && m.span_id != nullptr && m.in_span != nullptr;
  const unsigned chunks = spans ? 1u : unsigned(std::max(1, (m.T + 8191) / 8192));
  ListOut lo;
  lo.fwd = reinterpret_cast<uint32_t*>(plan + L.fwd_list);
  lo.dq = reinterpret_cast<uint32_t*>(plan + L.dq_list);
  lo.dkdv = reinterpret_cast<uint32_t*>(plan + L.dkdv_list);
  lo.fwd_n = reinterpret_cast<int32_t*>(plan + L.fwd_count);
  lo.dq_n = reinterpret_cast<int32_t*>(plan + L.dq_count);
  lo.dkdv_n = reinterpret_cast<int32_t*>(plan + L.dkdv_count);
  lo.fwd_order = reinterpret_cast<uint32_t*>(plan + L.fwd_order);
  lo.dq_order = reinterpret_cast<uint32_t*>(plan + L.dq_order);
  lo.dkdv_order = reinterpret_cast<uint32_t*>(plan + L.dkdv_order);
  lo.nqb = L.n_fwd_blocks;  // (the forward and dQ lists share the grouping of two q-tiles)
  lo.nkb = L.n_dkdv_blocks;
  hipLaunchKernelGGL(k_codes_rows, dim3(chunks, unsigned(m.B)), dim3(1024), 0, st, m, runs, run_sid, run_count, rep,
                     codes, lo.fwd_n, m.B * lo.nqb, lo.dkdv_n, m.B * lo.nkb);
  // k-tiles per wave: TM_KPW once the grid holds 2048 workgroups at that, else 1
  const int kpw = int64_t(m.B) * lo.nqb * ((L.nT + 2 * TM_KPW - 1) / (2 * TM_KPW)) >= 2048 ? TM_KPW : 1;
  hipLaunchKernelGGL(k_tilemap,
                     dim3(unsigned((L.nT + 2 * kpw - 1) / (2 * kpw)), unsigned(std::min(lo.nqb, 65535)),
                     unsigned(m.B)),
                     dim3(256), 0, st, codes, m.T, L.nT, kpw, lo.nqb, cls, nnz, lo.fwd_n, lo.dkdv_n, lo.nkb);
  hipLaunchKernelGGL(k_lists, dim3(unsigned(lo.nqb + lo.nkb), unsigned(m.B)), dim3(256), 0, st, cls, L.nT, lo);
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
