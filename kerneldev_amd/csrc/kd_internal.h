// Internal declarations shared by the kernel translation units and the C ABI.
#pragma once
#include <algorithm>

#include "../../include/kdattn.h"
#include "kd_common.h"

namespace kd {

typedef kd_meta_args MetaArgs;
typedef kd_attn_args AttnArgs;

enum : uint8_t { TILE_EMPTY = 0, TILE_PARTIAL = 1, TILE_FULL = 2 };

// The parts P and dS enter their products in (kd_attn_args.precision):
// KD_PREC_SINGLE 1, KD_PREC_SPLIT 2 (hi + lo), KD_PREC_SPLIT3 3 (hi + mid + lo)
inline int parts_of(int precision) {
  return precision == KD_PREC_SINGLE ? 1 : precision == KD_PREC_SPLIT3 ? 3 : 2;
}

// Block shapes of the attention kernels (rows per workgroup).  The plan's
// work lists group the 64x64 class map by these.
inline int fwd_rows_per_block(int /*D*/) { return 128; }
inline int dq_rows_per_block(int /*D*/) { return 128; }
inline int dkdv_keys_per_block(int /*D*/) { return 128; }

// Work-list entry: (tile << 8) | class of group member r in bits 2r..2r+1
// (r < 4: the row blocks of the list's group), so a wave reads its own
// member's class (FULL: no mask, EMPTY: nothing allowed, PARTIAL: bit masks).
KD_DEV inline uint32_t entry_tile(uint32_t e) { return e >> 8; }
KD_DEV inline uint32_t entry_class(uint32_t e, int r) { return (e >> (2 * r)) & 3u; }
KD_DEV inline bool entry_full(uint32_t e, int group) {
  return (e & 0xFFu) == (0xAAu & ((1u << (2 * group)) - 1u));
}

struct PlanLayout {
  size_t codes, rep, runs, run_sid, run_count, tok_in_span, tok_span_id, tok_prefix, cls, nnz, fwd_list, fwd_count, dq_list, dq_count, dkdv_list, dkdv_count,
      fwd_order, dq_order, dkdv_order, total;
  int nT, fwd_group, dq_group, dkdv_group, n_fwd_blocks, n_dq_blocks, n_dkdv_blocks;
};

PlanLayout plan_layout(int B, int T, int D);
int launch_plan(const MetaArgs& m, uint8_t* plan, hipStream_t st);
int launch_plan_tokens(const kd_token_args& t, uint8_t* plan, hipStream_t st);
int launch_tile_masks(const uint8_t* plan, int B, int T, int D, uint64_t* rows, uint64_t* cols, hipStream_t st);
int launch_mask_dense(const uint32_t* codes, int B, int H, int T, uint8_t* out, const int64_t* strides,
                      hipStream_t st);
int launch_fwd(const AttnArgs& a, const uint8_t* plan, hipStream_t st);
int launch_delta(const AttnArgs& a, hipStream_t st);
// fuse_delta: the dQ kernel also computes Delta and the LSE copy (k_delta's
// job) for its rows and stores them for the dK/dV kernel
int launch_dq(const AttnArgs& a, const uint8_t* plan, hipStream_t st, bool fuse_delta);
int launch_dkdv(const AttnArgs& a, const uint8_t* plan, hipStream_t st);
int launch_hadamard(const kd_rot_args& a, hipStream_t st);
int launch_quant(const kd_quant_args& a, hipStream_t st);
int launch_absmax(const kd_quant_args& a, float* amax, hipStream_t st);
int launch_span(const kd_span_args& a, hipStream_t st);
int launch_span_bwd(const kd_span_args& a, hipStream_t st);
// fp32 inputs (kd_simt.hip): Delta on the vector ALUs and the fp32 MFMA
// kernels; which: 0 forward, 1 Delta, 2 dQ, 3 dK/dV
bool use_simt(const AttnArgs& a);
int launch_simt_kernel(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st);
// fp32 attention at head dims 16 (on the 32 kernels), 32, 64, 128, 256 on the
// fp32 MFMA (kd_f32w.hip); which: 0 forward, 2 dQ, 3 dK/dV
int launch_f32mma(int which, const AttnArgs& a, const uint8_t* plan, hipStream_t st);
// Device address of the no-allocation workspace on the current device
// (kd_noalloc.hip); KD_OK, or a status with *err set.
int noalloc_workspace(float** out, const char** err);

}  // namespace kd

// The workgroup -> work item mappings (xcd_remap, fwd_work): plain integer
// code, host-callable too, so that a host program can check them
#define KD_WORK_FN __host__ __device__ inline
#include "kd_work.h"
