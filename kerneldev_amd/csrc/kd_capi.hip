// extern "C" entry points of libkdattn.so: argument checks, then launches.
// Every check that fails returns a status instead of launching, so a bad
// shape or stride never reaches a kernel.
#include <cmath>
#include <cstdio>
#include <string>

#include "kd_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* msg) {
  g_err = msg;
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool strides_ok(const int64_t* s) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] & 7) != 0) return false;
  return true;
}

// Largest element offset reachable by a [B, H, T, D] view (for int32 safety
// of the in-kernel index math the offsets are int64; this only rejects
// negative / overlapping-by-construction layouts).
int check_tensor(const void* p, const int64_t* s, const char* name, int T = 1, int D = 0, int esize = 2) {
  if (p == nullptr) {
    g_err = std::string(name) + " is NULL";
    return KD_ERR_INVALID;
  }
  if (!aligned16(p)) {
    g_err = std::string(name) + " must be 16-byte aligned";
    return KD_ERR_INVALID;
  }
  if (!strides_ok(s)) {
    g_err = std::string(name) + " strides (b, h, t) must be non-negative multiples of 8 elements";
    return KD_ERR_INVALID;
  }
  if (s[2] < D) {
    g_err = std::string(name) + " rows overlap: the t stride must be >= head_dim";
    return KD_ERR_INVALID;
  }
  // kernels address one (b, h) slice through a buffer resource of 32-bit size
  if (int64_t(T) * s[2] * esize >= (int64_t(1) << 31)) {
    g_err = std::string(name) + ": T * t_stride * element size must be < 2^31 bytes per (b, h) slice";
    return KD_ERR_UNSUPPORTED;
  }
  return KD_OK;
}

int check_common(const kd_attn_args* a) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B < 1 || a->H < 1 || a->T < 1) return fail(KD_ERR_INVALID, "B, H and T must be >= 1");
  if (a->T > (1 << 24) - 2) return fail(KD_ERR_UNSUPPORTED, "T must be < 2^24 - 1");
  if (int64_t(a->B) * a->H * ((a->T + 63) / 64) > (int64_t(1) << 31) - 1)
    return fail(KD_ERR_UNSUPPORTED, "B * H * ceil(T / 64) exceeds the grid limit");
  if (a->D != 16 && a->D != 32 && a->D != 64 && a->D != 128 && a->D != 256)
    return fail(KD_ERR_UNSUPPORTED, "head dim must be 16, 32, 64, 128 or 256");
  if (a->dtype != KD_BF16 && a->dtype != KD_F16 && a->dtype != KD_F32)
    return fail(KD_ERR_UNSUPPORTED, "dtype must be bf16, fp16 or fp32");
  if (a->dqk_signs != nullptr && (kd::use_simt(*a) || (a->D != 64 && a->D != 128)))
    return fail(KD_ERR_UNSUPPORTED, "dqk_signs is built for bf16 / fp16 at head dim 64 or 128");
  if (!(a->sm_scale > 0.f) || !std::isfinite(a->sm_scale))
    return fail(KD_ERR_INVALID, "sm_scale must be finite and > 0");
  if (a->precision != KD_PREC_SPLIT && a->precision != KD_PREC_SINGLE && a->precision != KD_PREC_SPLIT3)
    return fail(KD_ERR_INVALID, "precision must be KD_PREC_SPLIT, KD_PREC_SINGLE or KD_PREC_SPLIT3");
  return KD_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// O's rounding residual exists for 16-bit O only: the fp32 kernels neither
// write nor need it, and a stale buffer would enter Delta
int check_o_lo(const kd_attn_args* a) {
  if (a->o_lo == nullptr) return KD_OK;
  if (a->dtype == KD_F32) return fail(KD_ERR_INVALID, "o_lo is for bf16 / fp16 O; pass NULL with fp32 inputs");
  if (!aligned16(a->o_lo)) return fail(KD_ERR_INVALID, "o_lo must be 16-byte aligned");
  return KD_OK;
}

int esz(const kd_attn_args* a) { return a->dtype == KD_F32 ? 4 : 2; }

int check_span(const kd_span_args* a) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B < 1 || a->T < 1 || a->D < 1) return fail(KD_ERR_INVALID, "B, T and D must be >= 1");
  if (a->B > 65535) return fail(KD_ERR_UNSUPPORTED, "B must be <= 65535");
  if (a->D > 65536) return fail(KD_ERR_UNSUPPORTED, "D must be <= 65536");
  if (a->n_spans < 1 || a->n_spans > 8192) return fail(KD_ERR_UNSUPPORTED, "n_spans must be in 1 .. 8192");
  if (a->dtype != KD_BF16 && a->dtype != KD_F16) return fail(KD_ERR_UNSUPPORTED, "dtype must be bf16 or fp16");
  if (a->tokens_dtype != KD_I64 && a->tokens_dtype != KD_I32) return fail(KD_ERR_INVALID, "bad tokens dtype");
  if (a->tokens == nullptr || a->h == nullptr) return fail(KD_ERR_INVALID, "tokens and h are required");
  if (a->tokens_strides[0] < 0 || a->tokens_strides[1] < 0) return fail(KD_ERR_INVALID, "negative token strides");
  if (a->h_strides[0] < 0 || a->h_strides[1] < a->D) return fail(KD_ERR_INVALID, "bad h strides");
  return KD_OK;
}

// A plan buffer handed in by the caller: present, aligned, and at least as
// large as the layout of this shape needs (kd_plan_bytes).  The kernels index
// the plan by that layout, so a smaller buffer is refused here, on the host,
// before anything is launched.
int check_plan(const void* plan, int64_t plan_bytes, int B, int T, int D) {
  if (plan == nullptr) return fail(KD_ERR_INVALID, "plan is NULL");
  if (!aligned16(plan)) return fail(KD_ERR_INVALID, "plan must be 16-byte aligned");
  const int64_t need = int64_t(kd::plan_layout(B, T, D).total);
  if (plan_bytes < need) {
    g_err = "plan is " + std::to_string(plan_bytes) + " bytes; B = " + std::to_string(B) + ", T = " +
            std::to_string(T) + " needs " + std::to_string(need) + " (kd_plan_bytes)";
    return KD_ERR_INVALID;
  }
  return KD_OK;
}

}  // namespace

extern "C" {

int kd_version(void) { return 30300; }

const char* kd_last_error_string(void) { return g_err.c_str(); }

void kd_struct_sizes(size_t* meta, size_t* attn) {
  if (meta) *meta = sizeof(kd_meta_args);
  if (attn) *attn = sizeof(kd_attn_args);
}

void kd_struct_sizes2(size_t* rot, size_t* quant) {
  if (rot) *rot = sizeof(kd_rot_args);
  if (quant) *quant = sizeof(kd_quant_args);
}

void kd_struct_sizes3(size_t* tokens) {
  if (tokens) *tokens = sizeof(kd_token_args);
}

void kd_struct_sizes4(size_t* span) {
  if (span) *span = sizeof(kd_span_args);
}

int kd_span_scores(const kd_span_args* a, void* stream) {
  int r;
  if ((r = check_span(a))) return r;
  if (a->scores == nullptr || a->h_ctx == nullptr || a->h_spans == nullptr || a->span_lo == nullptr ||
      a->span_hi == nullptr || a->mask_pos == nullptr)
    return fail(KD_ERR_INVALID, "scores, h_ctx, h_spans, span_lo, span_hi and mask_pos are required");
  r = kd::launch_span(*a, as_stream(stream));
  return r ? fail(r, "kernel launch failed (span scores)") : KD_OK;
}

int kd_span_scores_bwd(const kd_span_args* a, void* stream) {
  int r;
  if ((r = check_span(a))) return r;
  if (a->dscores == nullptr || a->h_ctx == nullptr || a->h_spans == nullptr || a->span_lo == nullptr ||
      a->span_hi == nullptr || a->mask_pos == nullptr || a->dh == nullptr)
    return fail(KD_ERR_INVALID, "dscores, h_ctx, h_spans, span_lo, span_hi, mask_pos and dh are required");
  if (a->dh_strides[0] < 0 || a->dh_strides[1] < a->D) return fail(KD_ERR_INVALID, "bad dh strides");
  r = kd::launch_span_bwd(*a, as_stream(stream));
  return r ? fail(r, "kernel launch failed (span scores backward)") : KD_OK;
}

int kd_plan_build_tokens(const kd_token_args* t, void* plan, int64_t plan_bytes, void* stream) {
  if (t == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (t->B < 1 || t->T < 1) return fail(KD_ERR_INVALID, "B and T must be >= 1");
  if (t->T > (1 << 24) - 2) return fail(KD_ERR_UNSUPPORTED, "T must be < 2^24 - 1");
  if (t->B > 65535) return fail(KD_ERR_UNSUPPORTED, "B must be <= 65535");
  if (int r = check_plan(plan, plan_bytes, t->B, t->T, t->D)) return r;
  if (t->tokens == nullptr) return fail(KD_ERR_INVALID, "tokens is NULL");
  if (t->tokens_dtype != KD_I64 && t->tokens_dtype != KD_I32)
    return fail(KD_ERR_INVALID, "tokens dtype must be int64 or int32");
  if (t->rule != KD_RULE_COLLATE && t->rule != KD_RULE_FALLBACK && t->rule != KD_RULE_TEACHER)
    return fail(KD_ERR_INVALID, "unknown metadata rule");
  if (t->tokens_strides[0] < 0 || t->tokens_strides[1] < 0) return fail(KD_ERR_INVALID, "negative token strides");
  if (t->lens != nullptr && t->lens_stride < 0) return fail(KD_ERR_INVALID, "negative lens stride");
  const int r = kd::launch_plan_tokens(*t, static_cast<uint8_t*>(plan), as_stream(stream));
  return r ? fail(r, "kernel launch failed (plan from tokens)") : KD_OK;
}

int kd_quant_fp8(const kd_quant_args* a, void* stream) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B < 1 || a->H < 1 || a->T < 1) return fail(KD_ERR_INVALID, "B, H and T must be >= 1");
  if (a->D != 64 && a->D != 128 && a->D != 256)
    return fail(KD_ERR_UNSUPPORTED, "head dim must be 64, 128 or 256");
  if (a->dtype != KD_BF16 && a->dtype != KD_F16) return fail(KD_ERR_UNSUPPORTED, "dtype must be bf16 or fp16");
  if (a->amax == nullptr || a->scale == nullptr || a->y == nullptr)
    return fail(KD_ERR_INVALID, "amax, scale and y are required");
  if (!aligned16(a->y)) return fail(KD_ERR_INVALID, "y must be 16-byte aligned");
  int r;
  if ((r = check_tensor(a->x, a->x_strides, "x", a->T, a->D))) return r;
  r = kd::launch_quant(*a, as_stream(stream));
  return r ? fail(r, "kernel launch failed (quant)") : KD_OK;
}

int kd_absmax(const kd_quant_args* a, float* amax, void* stream) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B < 1 || a->H < 1 || a->T < 1) return fail(KD_ERR_INVALID, "B, H and T must be >= 1");
  if (a->D != 16 && a->D != 32 && a->D != 64 && a->D != 128 && a->D != 256)
    return fail(KD_ERR_UNSUPPORTED, "head dim must be 16, 32, 64, 128 or 256");
  if (a->dtype != KD_BF16 && a->dtype != KD_F16) return fail(KD_ERR_UNSUPPORTED, "dtype must be bf16 or fp16");
  if (amax == nullptr) return fail(KD_ERR_INVALID, "amax is required");
  int r;
  if ((r = check_tensor(a->x, a->x_strides, "x", a->T, a->D))) return r;
  r = kd::launch_absmax(*a, amax, as_stream(stream));
  return r ? fail(r, "kernel launch failed (absmax)") : KD_OK;
}

int kd_hadamard(const kd_rot_args* a, void* stream) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B < 1 || a->H < 1 || a->T < 1) return fail(KD_ERR_INVALID, "B, H and T must be >= 1");
  if (a->D != 16 && a->D != 32 && a->D != 64 && a->D != 128 && a->D != 256)
    return fail(KD_ERR_UNSUPPORTED, "head dim must be 16, 32, 64, 128 or 256");
  if (a->dtype != KD_BF16 && a->dtype != KD_F16 && a->dtype != KD_F32)
    return fail(KD_ERR_UNSUPPORTED, "dtype must be bf16, fp16 or fp32");
  if (a->signs == nullptr) return fail(KD_ERR_INVALID, "signs is NULL");
  if (int64_t(a->B) * a->H > 65535) return fail(KD_ERR_UNSUPPORTED, "B * H must be <= 65535");
  int r;
  const int es = a->dtype == KD_F32 ? 4 : 2;
  if ((r = check_tensor(a->x, a->x_strides, "x", a->T, a->D, es)) ||
      (r = check_tensor(a->y, a->y_strides, "y", a->T, a->D, es)))
    return r;
  if (a->x == a->y) return fail(KD_ERR_INVALID, "x and y must not alias");
  r = kd::launch_hadamard(*a, as_stream(stream));
  return r ? fail(r, "kernel launch failed (hadamard)") : KD_OK;
}

int64_t kd_plan_bytes(int32_t B, int32_t T, int32_t D) {
  if (B < 1 || T < 1) return -1;
  return int64_t(kd::plan_layout(B, T, D).total);
}

int kd_plan_layout(int32_t B, int32_t T, int32_t D, int64_t* off) {
  if (off == nullptr || B < 1 || T < 1) return fail(KD_ERR_INVALID, "bad plan_layout arguments");
  const kd::PlanLayout L = kd::plan_layout(B, T, D);
  const int64_t v[20] = {int64_t(L.codes),     int64_t(L.rep),        int64_t(L.cls),     int64_t(L.nnz),
                         int64_t(L.fwd_list),  int64_t(L.fwd_count),  int64_t(L.dq_list), int64_t(L.dq_count),
                         int64_t(L.dkdv_list), int64_t(L.dkdv_count), L.nT,               L.fwd_group,
                         L.dq_group,           L.dkdv_group,          L.n_fwd_blocks,     L.n_dq_blocks,
                         L.n_dkdv_blocks,      int64_t(L.fwd_order),  int64_t(L.dq_order), int64_t(L.dkdv_order)};
  for (int i = 0; i < 20; ++i) off[i] = v[i];
  return KD_OK;
}

int kd_plan_build(const kd_meta_args* m, void* plan, int64_t plan_bytes, void* stream) {
  if (m == nullptr) return fail(KD_ERR_INVALID, "meta is NULL");
  if (m->B < 1 || m->T < 1) return fail(KD_ERR_INVALID, "B and T must be >= 1");
  if (m->T > (1 << 24) - 2) return fail(KD_ERR_UNSUPPORTED, "T must be < 2^24 - 1");
  if (m->B > 65535) return fail(KD_ERR_UNSUPPORTED, "B must be <= 65535");
  if (int r = check_plan(plan, plan_bytes, m->B, m->T, m->D)) return r;
  if (m->mode != KD_MODE_FORMULA && m->mode != KD_MODE_CAUSAL && m->mode != KD_MODE_ALL)
    return fail(KD_ERR_INVALID, "unknown mask mode");
  if (m->span_id != nullptr && m->span_id_dtype != KD_I64 && m->span_id_dtype != KD_I32)
    return fail(KD_ERR_INVALID, "span_id dtype must be int64 or int32");
  const int64_t* ss[3] = {m->in_span_strides, m->span_id_strides, m->is_prefix_strides};
  for (int i = 0; i < 3; ++i)
    if (ss[i][0] < 0 || ss[i][1] < 0) return fail(KD_ERR_INVALID, "metadata strides must be non-negative");
  return kd::launch_plan(*m, static_cast<uint8_t*>(plan), as_stream(stream));
}

static int check_fp8(const kd_attn_args* a) {
  if ((a->q8 == nullptr) != (a->k8 == nullptr)) return fail(KD_ERR_INVALID, "q8 and k8 go together");
  if (a->q8 == nullptr) return KD_OK;
  if (a->precision == KD_PREC_SPLIT3)
    return fail(KD_ERR_UNSUPPORTED, "KD_PREC_SPLIT3 is not built with fp8 scores");
  if (a->D != 64 && a->D != 128 && a->D != 256)
    return fail(KD_ERR_UNSUPPORTED, "the fp8 QK^T path is built for head dims 64, 128 and 256");
  if (a->dtype != KD_BF16) return fail(KD_ERR_UNSUPPORTED, "the fp8 QK^T path is built for bf16");
  if (!aligned16(a->q8) || !aligned16(a->k8)) return fail(KD_ERR_INVALID, "q8 and k8 must be 16-byte aligned");
  if (a->q_scale == nullptr || a->k_scale == nullptr) return fail(KD_ERR_INVALID, "q_scale and k_scale are required");
  return KD_OK;
}

int kd_attn_fwd(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  int r = check_common(a);
  if (r) return r;
  if ((r = check_fp8(a))) return r;
  if ((r = check_plan(plan, plan_bytes, a->B, a->T, a->D))) return r;
  if ((r = check_tensor(a->q, a->q_strides, "q", a->T, a->D, esz(a))) || (r = check_tensor(a->k, a->k_strides, "k", a->T, a->D, esz(a))) ||
      (r = check_tensor(a->v, a->v_strides, "v", a->T, a->D, esz(a))) || (r = check_tensor(a->o, a->o_strides, "o", a->T, a->D, esz(a))))
    return r;
  if ((r = check_o_lo(a))) return r;
  r = kd::launch_fwd(*a, static_cast<const uint8_t*>(plan), as_stream(stream));
  return r ? fail(r, "kernel launch failed (forward)") : KD_OK;
}

int kd_attn_bwd_delta(const kd_attn_args* a, void* stream) {
  int r = check_common(a);
  if (r) return r;
  if ((r = check_tensor(a->o, a->o_strides, "o", a->T, a->D, esz(a))) || (r = check_tensor(a->dout, a->do_strides, "dout", a->T, a->D, esz(a))))
    return r;
  if (a->delta == nullptr || a->lse == nullptr) return fail(KD_ERR_INVALID, "delta and lse are required");
  if ((r = check_o_lo(a))) return r;
  r = kd::launch_delta(*a, as_stream(stream));
  return r ? fail(r, "kernel launch failed (delta)") : KD_OK;
}

// own_workspace: the library provides a->delta (kd_attn_bwd_noalloc)
static int check_bwd(const kd_attn_args* a, const void* plan, int64_t plan_bytes, bool own_workspace = false) {
  int r = check_common(a);
  if (r) return r;
  if ((r = check_fp8(a))) return r;
  if ((r = check_plan(plan, plan_bytes, a->B, a->T, a->D))) return r;
  if (a->lse == nullptr || (a->delta == nullptr && !own_workspace))
    return fail(KD_ERR_INVALID, "lse and delta are required");
  if (a->dq_lo != nullptr || a->dk_lo != nullptr || a->dv_lo != nullptr) {
    if (kd::use_simt(*a) || a->dqk_signs != nullptr)
      return fail(KD_ERR_UNSUPPORTED, "dq_lo / dk_lo / dv_lo are built for bf16 / fp16 inputs, without dqk_signs");
    for (const void* p : {a->dq_lo, a->dk_lo, a->dv_lo})
      if (p != nullptr && !aligned16(p)) return fail(KD_ERR_INVALID, "dq_lo, dk_lo and dv_lo must be 16-byte aligned");
  }
  if ((r = check_tensor(a->q, a->q_strides, "q", a->T, a->D, esz(a))) || (r = check_tensor(a->k, a->k_strides, "k", a->T, a->D, esz(a))) ||
      (r = check_tensor(a->v, a->v_strides, "v", a->T, a->D, esz(a))) || (r = check_tensor(a->dout, a->do_strides, "dout", a->T, a->D, esz(a))))
    return r;
  return KD_OK;
}

int kd_attn_bwd_dq(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  int r = check_bwd(a, plan, plan_bytes);
  if (r) return r;
  if ((r = check_tensor(a->dq, a->dq_strides, "dq", a->T, a->D, esz(a)))) return r;
  r = kd::launch_dq(*a, static_cast<const uint8_t*>(plan), as_stream(stream), false);
  return r ? fail(r, "kernel launch failed (dq)") : KD_OK;
}

int kd_attn_bwd_dkdv(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  int r = check_bwd(a, plan, plan_bytes);
  if (r) return r;
  if ((r = check_tensor(a->dk, a->dk_strides, "dk", a->T, a->D, esz(a))) || (r = check_tensor(a->dv, a->dv_strides, "dv", a->T, a->D, esz(a)))) return r;
  r = kd::launch_dkdv(*a, static_cast<const uint8_t*>(plan), as_stream(stream));
  return r ? fail(r, "kernel launch failed (dkdv)") : KD_OK;
}

int kd_attn_bwd_dq_delta(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  int r = check_bwd(a, plan, plan_bytes);
  if (r) return r;
  if ((r = check_tensor(a->o, a->o_strides, "o", a->T, a->D, esz(a))) || (r = check_tensor(a->dq, a->dq_strides, "dq", a->T, a->D, esz(a))))
    return r;
  if ((r = check_o_lo(a))) return r;
  r = kd::launch_dq(*a, static_cast<const uint8_t*>(plan), as_stream(stream), true);
  return r ? fail(r, "kernel launch failed (dq)") : KD_OK;
}

// Every check of kd_attn_bwd_dq_delta and kd_attn_bwd_dkdv, so that the
// whole backward is refused before either half is launched.
static int check_bwd_all(const kd_attn_args* a, const void* plan, int64_t plan_bytes, bool own_workspace = false) {
  int r = check_bwd(a, plan, plan_bytes, own_workspace);
  if (r) return r;
  if ((r = check_tensor(a->o, a->o_strides, "o", a->T, a->D, esz(a))) ||
      (r = check_tensor(a->dq, a->dq_strides, "dq", a->T, a->D, esz(a))) ||
      (r = check_tensor(a->dk, a->dk_strides, "dk", a->T, a->D, esz(a))) ||
      (r = check_tensor(a->dv, a->dv_strides, "dv", a->T, a->D, esz(a))))
    return r;
  return check_o_lo(a);
}

int kd_attn_bwd(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  int r = check_bwd_all(a, plan, plan_bytes);
  if (r) return r;
  r = kd_attn_bwd_dq_delta(a, plan, plan_bytes, stream);
  return r ? r : kd_attn_bwd_dkdv(a, plan, plan_bytes, stream);
}

int kd_attn_bwd_noalloc(const kd_attn_args* a, const void* plan, int64_t plan_bytes, void* stream) {
  if (a == nullptr) return fail(KD_ERR_INVALID, "args is NULL");
  if (a->B >= 1 && a->H >= 1 && a->T >= 1 &&
      2 * int64_t(a->B) * a->H * a->T > int64_t(KD_NOALLOC_WORKSPACE_FLOATS))
    return fail(KD_ERR_UNSUPPORTED,
                "kd_attn_bwd_noalloc: B * H * T exceeds the workspace (KD_NOALLOC_WORKSPACE_FLOATS / 2 rows)");
  int r = check_bwd_all(a, plan, plan_bytes, true);  // every refusal before the device is touched
  if (r) return r;
  kd_attn_args w = *a;
  const char* err = nullptr;
  float* ws = nullptr;
  r = kd::noalloc_workspace(&ws, &err);
  if (r) return fail(r, err);
  w.delta = ws;
  return kd_attn_bwd(&w, plan, plan_bytes, stream);
}

int kd_tile_masks(const void* plan, int64_t plan_bytes, int32_t B, int32_t T, int32_t D, uint64_t* rows,
                  uint64_t* cols, void* stream) {
  if (rows == nullptr || cols == nullptr) return fail(KD_ERR_INVALID, "NULL argument");
  if (B < 1 || T < 1) return fail(KD_ERR_INVALID, "B and T must be >= 1");
  // (one workgroup row per q-tile: the grid's y extent holds at most 65535)
  if (T > 65535 * 64) return fail(KD_ERR_UNSUPPORTED, "kd_tile_masks takes T <= 65535 * 64");
  if (B > 65535) return fail(KD_ERR_UNSUPPORTED, "B must be <= 65535");
  if (int r = check_plan(plan, plan_bytes, B, T, D)) return r;
  const int r = kd::launch_tile_masks(static_cast<const uint8_t*>(plan), B, T, D, rows, cols, as_stream(stream));
  return r ? fail(r, "kernel launch failed (tile masks)") : KD_OK;
}

int kd_mask_dense(const void* plan, int64_t plan_bytes, int32_t B, int32_t H, int32_t T, int32_t D, uint8_t* out,
                  const int64_t* strides, void* stream) {
  if (out == nullptr || strides == nullptr) return fail(KD_ERR_INVALID, "NULL argument");
  if (B < 1 || H < 1 || T < 1) return fail(KD_ERR_INVALID, "B, H and T must be >= 1");
  if (T > (1 << 24) - 2) return fail(KD_ERR_UNSUPPORTED, "T must be < 2^24 - 1");
  if (int r = check_plan(plan, plan_bytes, B, T, D)) return r;
  for (int i = 0; i < 4; ++i)
    if (strides[i] < 0) return fail(KD_ERR_INVALID, "mask strides must be non-negative");
  const kd::PlanLayout L = kd::plan_layout(B, T, D);
  const uint32_t* codes = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(plan) + L.codes);
  const int r = kd::launch_mask_dense(codes, B, H, T, out, strides, as_stream(stream));
  return r ? fail(r, "kernel launch failed (mask)") : KD_OK;
}

}  // extern "C"
