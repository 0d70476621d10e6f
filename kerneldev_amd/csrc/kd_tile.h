// LDS tile primitives for the gfx950 attention kernels.
//
// A "tile" is 64 rows (keys or queries) x D columns of 16-bit elements,
// stored row-major in LDS (D * 2 bytes per row) and filled straight from
// global memory with buffer_load ... lds (no VGPR staging, no VALU).  Rows
// at or beyond T read as zero: every global access goes through a buffer
// resource whose size ends at row T, so there are no per-lane branches.
//
// Bank-conflict-free layout: the 16-byte chunk c of row r is stored at chunk
// position c ^ swz(r).  swz is chosen so that both read patterns the kernels
// use are conflict free:
//   (a) ds_read_b128 of one chunk from 16 different rows (an MFMA A operand
//       taken row-wise: 16 lanes, 16 rows r0..r0+15 in any order);
//   (b) ds_read_b64_tr_b16 of a 4-row x 32-column block by 32 lanes (an MFMA
//       A operand taken column-wise, i.e. the tile transposed on the fly).
// For D = 128 (16 chunks per 256-byte row) swz(r) = 4 (r & 3) + ((r >> 2) & 3);
// for D = 64 (8 chunks per 128-byte row, two rows per bank sweep)
// swz(r) = 4 ((r >> 1) & 1) + ((r >> 2) & 3).
#pragma once
#include <type_traits>

#include "kd_internal.h"

namespace kd {

typedef __attribute__((address_space(3))) void lds_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes); word 3 as for every gfx9 part.
KD_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

KD_DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// A byte offset that no buffer resource here reaches (they all end below
// 2^31 bytes, which the C ABI checks), also after a tile offset < 2^31 is
// added: a load from it returns zeros, a DMA writes zeros to LDS.
constexpr uint32_t OFF_OUTSIDE = 0x80000000u;

// Head dims 16 and 32 run on the D = 64 kernels: each row holds dbytes =
// 2 D_real bytes and the columns from there to 64 are read as zeros, by
// sending the loads of those 16-byte chunks outside the buffer.  col: the
// chunk's byte offset within the row.
KD_DEV uint32_t col_masked(uint32_t off, uint32_t col, uint32_t dbytes) { return col < dbytes ? off : OFF_OUTSIDE; }

// make_rsrc's four descriptor words, for the inline-asm loads below
KD_DEV u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  auto u = [](uint32_t x) { return uint32_t(__builtin_amdgcn_readfirstlane(int(x))); };
  return u32x4{u(uint32_t(a)), u(uint32_t(a >> 32) & 0xFFFFu), u(bytes), 0x00020000u};
}

// One wave-wide global -> LDS copy of 16 bytes per lane (buffer_load_dwordx4
// ... lds, LDS address m0 + 16 lane) issued as inline asm.  Through the
// builtin, the compiler treats LDS as written by a load in flight and makes
// every later LDS read wait for all outstanding loads (s_waitcnt vmcnt(0)),
// which drains tile prefetches meant to stay in flight for longer.  Hidden
// from the compiler, the copies are ordered by the caller: wait_vmem_n /
// wait_vmem before barrier_raw, and no copy into a slot until every wave has
// passed the barrier after its last read of that slot.  The s_nop gives the
// wait states an LDS DMA needs after an SALU write of m0 (1) and after a VALU
// write (v_readfirstlane) of an SGPR it reads (5), which the compiler's hazard
// check does not see inside the asm.
KD_DEV void dma_b128(const u32x4& rs, uint32_t voff, uint32_t m0v) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "s"(m0v)
               : "memory", "m0");
}

template <int D, int NW = 4>  // NW: waves that share the copy of one tile
struct Tile {
  static constexpr int ROWS = 64;
  static constexpr int ROWB = D * 2;            // bytes per row
  static constexpr int CPR = D / 8;             // 16-byte chunks per row
  static constexpr int BYTES = ROWS * ROWB;     // 16 KiB (D = 128) or 8 KiB (D = 64)
  static constexpr int LOADS = BYTES / 1024;    // 1 KiB per wave-wide buffer_load_dwordx4
  static constexpr int LOADS_PER_WAVE = LOADS / NW;
  static_assert(LOADS % NW == 0, "tile copy must split evenly over the waves");

  KD_DEV static int swz(int r) {
    // D = 256: 512-byte rows meet the banks as 256-byte rows do, so the
    // D = 128 swizzle (low four chunk bits) serves them too.  D = 32 (64-byte
    // rows: the fp8 tiles at head dim 64): the 16 rows a half-wave reads fill
    // the 256 bytes of banks 4 times over, rows r and r + 4 k sharing their
    // bank offset, so their chunks are told apart by row bits 2 and 3
    if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else if constexpr (D == 32) return (r >> 2) & 3;
    else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  }
  // byte offset of (row, 16-byte chunk) inside the tile
  KD_DEV static int at(int r, int chunk) { return r * ROWB + ((chunk ^ swz(r)) << 4); }

  // Per-lane global byte offsets (relative to the tile's first row) of the
  // chunks this lane moves in each of its LOADS_PER_WAVE wave-wide loads.
  // Columns from dbytes on (rows narrower than the tile) read as zeros.
  KD_DEV static void load_offsets(int wave, int lane, uint32_t row_bytes, uint32_t (&off)[LOADS_PER_WAVE],
                                  uint32_t dbytes = ROWB) {
#pragma unroll
    for (int j = 0; j < LOADS_PER_WAVE; ++j) {
      const int u = (wave * LOADS_PER_WAVE + j) * 64 + lane;  // LDS chunk index, row-major
      const int r = u / CPR, pos = u % CPR;
      const int chunk = pos ^ swz(r);
      off[j] = col_masked(uint32_t(r) * row_bytes + uint32_t(chunk) * 16u, uint32_t(chunk) * 16u, dbytes);
    }
  }
  // This wave's share of the tile load through dma_b128 (invisible to the
  // compiler's wait insertion; see there).  lds_tile: LDS byte address.
  KD_DEV static void load_async(const u32x4& rs, uint32_t tile_off, const uint32_t (&off)[LOADS_PER_WAVE],
                                uint32_t lds_tile, int wave) {
    const uint32_t m = uint32_t(__builtin_amdgcn_readfirstlane(int(lds_tile + uint32_t(wave * LOADS_PER_WAVE) * 1024u)));
#pragma unroll
    for (int j = 0; j < LOADS_PER_WAVE; ++j) dma_b128(rs, off[j] + tile_off, m + uint32_t(j) * 1024u);
  }
  // The same copy with two per-lane registers instead of LOADS_PER_WAVE.  The
  // rows of a wave's load j are those of its load 0 plus j RPL.  The wave's
  // first row, j RPL and the lane's row within a load (lane / CPR) occupy
  // disjoint bits, and swz is an XOR of selected row bits, so the swizzle of
  // load j's row splits into a per-lane part (in c16) and a constant per j:
  //   source offset of load j = arow + j RPL row_bytes + (c16 ^ swz(j RPL) << 4)
  // with arow = lane_row(wave, lane) * row_bytes, c16 = lane_chunk16(wave, lane).
  // (Everything stays in the VGPR offset, which the buffer's range check
  // covers, so rows past the end still read as zero.)
  static constexpr int RPL = 64 / CPR;  // rows per wave-wide load
  KD_DEV static uint32_t lane_row(int wave, int lane) { return uint32_t(wave * LOADS_PER_WAVE * RPL + lane / CPR); }
  KD_DEV static uint32_t lane_chunk16(int wave, int lane) {
    return uint32_t(((lane % CPR) ^ swz(lane / CPR) ^ swz(wave * LOADS_PER_WAVE * RPL)) << 4);
  }
  KD_DEV static void load_async_rows(const u32x4& rs, uint32_t tile_off, uint32_t arow, uint32_t c16,
                                     uint32_t row_bytes, uint32_t lds_tile, int wave) {
    const uint32_t m = uint32_t(__builtin_amdgcn_readfirstlane(int(lds_tile + uint32_t(wave * LOADS_PER_WAVE) * 1024u)));
#pragma unroll
    for (int j = 0; j < LOADS_PER_WAVE; ++j)
      dma_b128(rs, arow + (tile_off + uint32_t(j * RPL) * row_bytes) + (c16 ^ uint32_t(swz(j * RPL) << 4)),
               m + uint32_t(j) * 1024u);
  }
  // Issue this wave's share of the tile load (asynchronous; vmcnt tracks it).
  KD_DEV static void load(__amdgpu_buffer_rsrc_t rs, uint32_t tile_off, const uint32_t (&off)[LOADS_PER_WAVE],
                          uint8_t* lds_tile, int wave) {
#pragma unroll
    for (int j = 0; j < LOADS_PER_WAVE; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_t*)(lds_tile + (wave * LOADS_PER_WAVE + j) * 1024), 16, off[j] + tile_off, 0, 0, 0);
  }
};

// 32 lanes of one half-wave exchange with the other half: returns op(x, x of lane ^ 32).
KD_DEV float xhalf_max(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
KD_DEV float xhalf_sum(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Transposed 4x16 read: lane i of each 16-lane group gets column (i) of the
// 4 rows addressed by the group (see Tile layout); 4 x 16-bit per lane.
KD_DEV u32x2 ds_read_tr16(const uint8_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Pointers into LDS typed as such: offsets added to them stay 32-bit LDS
// addresses (a register plus the instruction's immediate offset), where a
// generic pointer is converted back to LDS after every addition.
typedef const __attribute__((address_space(3))) uint8_t lds_u8;
KD_DEV lds_u8* to_lds(const uint8_t* p) { return (lds_u8*)(p); }
KD_DEV u32x2 ds_read_tr16(lds_u8* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(u32x2, v);
}
KD_DEV u32x4 ds_read16(lds_u8* p) { return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(p); }

// LDS byte address of a pointer into __shared__ memory
KD_DEV uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)(p)));
}

// dma_b128's 4-byte form: lane i copies 4 bytes to LDS address m0 + 4 i
KD_DEV void dma_b32(const u32x4& rs, uint32_t voff, uint32_t m0v) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "s"(m0v)
               : "memory", "m0");
}

// s_barrier without the release/acquire fences of __syncthreads(): those make
// the compiler wait for every outstanding load first (s_waitcnt vmcnt(0)),
// including tile loads meant to stay in flight across the barrier.  The caller
// orders memory itself: it has consumed its own LDS reads and waited (with
// wait_vmem / wait_vmem_n) for the loads other waves will read.
KD_DEV void barrier_raw() { asm volatile("s_barrier" ::: "memory"); }
// barrier_raw that first completes this wave's LDS writes (s_waitcnt
// lgkmcnt(0)), for steps where waves hand data to each other through LDS
KD_DEV void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Ends the compiler's tracking of a load into v: placed where the load is
// known complete (after wait_vmem), the compiler puts its own wait for it
// here, and none at later uses.
template <class T>
KD_DEV void settle(T& v) { asm volatile("" : "+v"(v)); }

// The lane index, computed where it is used (two VALU ops).  Values derived
// from the lane and needed only on rare paths of a step loop (a PARTIAL
// tile's mask) are better recomputed from this than kept live: at the
// kernels' register budget the compiler spills them, and a spill reload in
// the loop carries an s_waitcnt vmcnt(0) that also waits for the tile copies
// in flight.  Being volatile, it is neither hoisted nor merged with the
// prologue's lane index.
KD_DEV int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

KD_DEV void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// wait until at most N vector memory loads of this wave are outstanding
template <int N>
KD_DEV void wait_vmem_n() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

typedef int i32x8 __attribute__((ext_vector_type(8)));

// The score product S = X Y^T of one 64-row LDS tile (A operand, rows = the
// tile's tokens, taken sigma-permuted so the 32x32 output feeds the next MFMA
// as its B operand) against one register-resident row per lane (B operand).
//   Q8 = false: 16-bit X and Y, v_mfma_f32_32x32x16, D / 16 k-steps.
//   Q8 = true:  fp8 e4m3 X and Y (D bytes per row), v_mfma_scale_f32_32x32x64
//               f8f6f4 with unit block scales, D / 64 k-steps; the caller
//               applies the per-(b, h) dequantisation scales.
// In both, lane (c, hf) of an operand holds row c and the k-slots of half hf
// of each k-step, so the register row and the LDS row are read alike.
template <class E, int D, bool Q8>
struct ScoreOp;

template <class E, int D>
struct ScoreOp<E, D, false> {
  using TL = Tile<D>;
  using A = u32x4;  // one k-step's A operand
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int NK = D / 16;
  u32x4 b[NK];
  int addr[NK];
  // k-step st of rows 32 kb + sigma(c): read it, then multiply it in
  KD_DEV A read_a(const uint8_t* tile, int kb, int st) const {
    return *reinterpret_cast<const u32x4*>(tile + addr[st] + kb * 32 * TL::ROWB);
  }
  KD_DEV f32x16 mma_a(const A& a, int st, const f32x16& c) const { return mfma32x32x16<E>(a, b[st], c); }
  // dbytes: the row's bytes (2 D_real); columns from there on read as zeros
  KD_DEV void load_b(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, int hf, uint32_t dbytes = ROW_BYTES) {
#pragma unroll
    for (int st = 0; st < NK; ++st) {
      const uint32_t col = (16 * st + 8 * hf) * 2;
      b[st] = buf_load16(rs, col_masked(row_off + col, col, dbytes));
    }
  }
  KD_DEV void init(int srow, int hf) {
#pragma unroll
    for (int st = 0; st < NK; ++st) addr[st] = TL::at(srow, 2 * st + hf);
  }
  // Call once load_b's loads are known complete (after a wait_vmem): from
  // here on the compiler treats b as plain registers and places no wait for
  // them later, where it cannot see that no load is pending (the inline-asm
  // tile copies are invisible to it, so it would wait for those too).
  KD_DEV void settle() {
#pragma unroll
    for (int st = 0; st < NK; ++st) asm volatile("" : "+v"(b[st]));
  }
};

template <class E, int D>
struct ScoreOp<E, D, true> {
  using TL = Tile<D / 2>;  // D bytes per row, laid out as D/2 16-bit columns
  using A = i32x8;
  static constexpr int ROW_BYTES = D;
  static constexpr int NK = D / 64;
  i32x8 b[NK];
  int addr[NK][2];
  KD_DEV A read_a(const uint8_t* tile, int kb, int st) const {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + addr[st][0] + kb * 32 * TL::ROWB);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + addr[st][1] + kb * 32 * TL::ROWB);
    return i32x8{int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]), int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
  }
  KD_DEV f32x16 mma_a(const A& a, int st, const f32x16& c) const {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b[st], c, 0, 0, 0, 127, 0, 127);
  }
  KD_DEV void load_b(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, int hf, uint32_t /*dbytes*/ = ROW_BYTES) {
#pragma unroll
    for (int st = 0; st < NK; ++st) {
      const u32x4 lo = buf_load16(rs, row_off + 64 * st + 32 * hf);
      const u32x4 hi = buf_load16(rs, row_off + 64 * st + 32 * hf + 16);
      b[st] = i32x8{int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]), int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
    }
  }
  KD_DEV void init(int srow, int hf) {
#pragma unroll
    for (int st = 0; st < NK; ++st) {
      addr[st][0] = TL::at(srow, 4 * st + 2 * hf);
      addr[st][1] = TL::at(srow, 4 * st + 2 * hf + 1);
    }
  }
  KD_DEV void settle() {
#pragma unroll
    for (int st = 0; st < NK; ++st) asm volatile("" : "+v"(b[st]));
  }
};

// Sum of a packed pair of 16-bit floats into an fp32 accumulator (v_dot2).
template <class E> KD_DEV float acc_pair(uint32_t w, float acc);
template <> KD_DEV float acc_pair<BF16>(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
}
template <> KD_DEV float acc_pair<F16>(uint32_t w, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
}

}  // namespace kd
