/*
 * A C caller of libkdattn.so, with no Python or torch: plan, forward and
 * backward through include/kdattn.h on HIP device buffers, checked against a
 * double-precision CPU attention written here.  The causal, no-metadata
 * case is the reference's teacher-forcing mode (original_kernel.py:512-513).
 * A second leg runs the fp8 e4m3 score path through the same boundary:
 * kd_absmax and kd_quant_fp8 make the e4m3 copies of Q and K, and the
 * attention takes them in q8 / k8; its reference takes the scores from the
 * decoded e4m3 bytes times the scales and the gradients straight through
 * the bf16 Q and K.
 * tests/test_gpu_c_abi.py runs it; the build step compiles it with gcc
 * against the HIP runtime's C API.
 *
 * Exit status 0 when O, LSE, dQ, dK and dV match (max-abs 2e-2 beyond one
 * bf16 ulp, as the Python parity tests), 1 on a mismatch, 2 on an API error.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kdattn.h"

enum { B = 2, H = 2, T = 200, D = 64 };
#define N ((size_t)B * H * T * D)

static uint16_t to_bf16(float f) { /* round to nearest even */
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint64_t rng = 0x9E3779B97F4A7C15ull;
static double uniform(void) {
  rng = rng * 6364136223846793005ull + 1442695040888963407ull;
  return ((rng >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static float normal(void) { return (float)(sqrt(-2.0 * log(uniform())) * cos(6.283185307179586 * uniform())); }

#define HIP_OK(x)                                                      \
  do {                                                                 \
    if ((x) != hipSuccess) {                                           \
      fprintf(stderr, "HIP error at %s:%d\n", __FILE__, __LINE__);     \
      return 2;                                                        \
    }                                                                  \
  } while (0)
#define KD_OK_OR_FAIL(x, what)                                                     \
  do {                                                                             \
    int st_ = (x);                                                                 \
    if (st_ != KD_OK) {                                                            \
      fprintf(stderr, "%s: status %d (%s)\n", what, st_, kd_last_error_string()); \
      return 2;                                                                    \
    }                                                                              \
  } while (0)

/* OCP e4m3: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is subnormal */
static float from_e4m3(uint8_t b) {
  const int e = (b >> 3) & 15, m = b & 7;
  const float mag = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + m / 8.0f, e - 7);
  return (b & 0x80) ? -mag : mag;
}

/* max |got - want| beyond one bf16 ulp of want */
static double excess(const float* got, const double* want, size_t n, double* maxabs) {
  double worst = 0.0;
  *maxabs = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double e = fabs((double)got[i] - want[i]);
    const double ulp = want[i] == 0.0 ? 0.0 : ldexp(1.0, ilogb(want[i]) - 7);
    if (e > *maxabs) *maxabs = e;
    if (e - ulp > worst) worst = e - ulp;
  }
  return worst;
}

/* Double-precision causal attention, forward and backward, into the outputs'
 * references: the scores from sq . sk (Q and K themselves, or their decoded
 * e4m3 copies times the scales), P V and the gradients dQ = dS K, dK = dS^T Q
 * from the bf16 values x = {Q, K, V, dO}.  Returns 1 on a mismatch. */
static int check(const char* leg, float* const x[4], const float* sq, const float* sk, float* const got[4],
                 const float* lse) {
  const double scale = 0.125; /* 1 / sqrt(64) */
  double *ro = calloc(N, 8), *rdq = calloc(N, 8), *rdk = calloc(N, 8), *rdv = calloc(N, 8);
  double *rl = calloc((size_t)B * H * T, 8), *p = malloc(sizeof(double) * T), *dp = malloc(sizeof(double) * T);
  for (int bh = 0; bh < B * H; ++bh) {
    const size_t base = (size_t)bh * T * D;
    const float *q = x[0] + base, *k = x[1] + base, *v = x[2] + base, *g = x[3] + base;
    const float *qs = sq + base, *ks = sk + base;
    for (int i = 0; i < T; ++i) {
      double mx = -INFINITY, sum = 0.0;
      for (int j = 0; j <= i; ++j) {
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)qs[i * D + d] * ks[j * D + d];
        p[j] = s * scale;
        if (p[j] > mx) mx = p[j];
      }
      for (int j = 0; j <= i; ++j) sum += (p[j] = exp(p[j] - mx));
      rl[(size_t)bh * T + i] = (mx + log(sum)) / log(2.0);
      double delta_i = 0.0;
      for (int j = 0; j <= i; ++j) p[j] /= sum;
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int j = 0; j <= i; ++j) acc += p[j] * v[j * D + d];
        ro[base + (size_t)i * D + d] = acc;
        delta_i += acc * g[i * D + d];
      }
      for (int j = 0; j <= i; ++j) {
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)g[i * D + d] * v[j * D + d];
        dp[j] = p[j] * (s - delta_i); /* dS */
        for (int d = 0; d < D; ++d) {
          rdv[base + (size_t)j * D + d] += p[j] * g[i * D + d];
          rdk[base + (size_t)j * D + d] += dp[j] * scale * q[i * D + d];
          rdq[base + (size_t)i * D + d] += dp[j] * scale * k[j * D + d];
        }
      }
    }
  }
  const char* names[4] = {"O", "dQ", "dK", "dV"};
  double* refs[4] = {ro, rdq, rdk, rdv};
  int bad = 0;
  for (int i = 0; i < 4; ++i) {
    double mabs;
    const double ex = excess(got[i], refs[i], N, &mabs);
    printf("%s %s: max_abs %.3e, beyond one bf16 ulp %.3e\n", leg, names[i], mabs, ex);
    if (!(ex <= 2e-2)) bad = 1;
  }
  double lerr = 0.0;
  for (size_t i = 0; i < (size_t)B * H * T; ++i) lerr = fmax(lerr, fabs(lse[i] - rl[i]));
  printf("%s LSE (log2): max_abs %.3e\n", leg, lerr);
  if (!(lerr <= 1e-3)) bad = 1;
  free(ro), free(rdq), free(rdk), free(rdv), free(rl), free(p), free(dp);
  return bad;
}

int main(void) {
  const float scale = 0.125f; /* 1 / sqrt(64) */
  uint16_t *hq = malloc(N * 2), *hk = malloc(N * 2), *hv = malloc(N * 2), *hdo = malloc(N * 2), *hbuf = malloc(N * 2);
  float *x[4], *got[4], *lse = malloc(sizeof(float) * B * H * T);
  for (int i = 0; i < 4; ++i) {
    x[i] = malloc(N * sizeof(float));
    got[i] = malloc(N * sizeof(float));
  }
  uint16_t* hx[4] = {hq, hk, hv, hdo};
  for (int i = 0; i < 4; ++i)
    for (size_t j = 0; j < N; ++j) {
      hx[i][j] = to_bf16(normal());
      x[i][j] = from_bf16(hx[i][j]); /* the reference sees the rounded inputs */
    }

  /* the error path needs no GPU: a NULL argument struct is refused */
  if (kd_attn_fwd(NULL, NULL, 0, NULL) != KD_ERR_INVALID || strlen(kd_last_error_string()) == 0) {
    fprintf(stderr, "NULL args were not refused\n");
    return 1;
  }

  void *dq_, *dk_, *dv_, *dd_, *o, *olo, *dq, *dk, *dv, *plan;
  float *dlse, *delta;
  HIP_OK(hipMalloc(&dq_, N * 2));
  HIP_OK(hipMalloc(&dk_, N * 2));
  HIP_OK(hipMalloc(&dv_, N * 2));
  HIP_OK(hipMalloc(&dd_, N * 2));
  HIP_OK(hipMalloc(&o, N * 2));
  HIP_OK(hipMalloc(&olo, N * 2));
  HIP_OK(hipMalloc(&dq, N * 2));
  HIP_OK(hipMalloc(&dk, N * 2));
  HIP_OK(hipMalloc(&dv, N * 2));
  HIP_OK(hipMalloc((void**)&dlse, sizeof(float) * B * H * T));
  HIP_OK(hipMalloc((void**)&delta, sizeof(float) * 2 * B * H * T));
  const int64_t pbytes = kd_plan_bytes(B, T, D);
  if (pbytes <= 0) return 2;
  HIP_OK(hipMalloc(&plan, (size_t)pbytes));
  HIP_OK(hipMemcpy(dq_, hq, N * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dk_, hk, N * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dv_, hv, N * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dd_, hdo, N * 2, hipMemcpyHostToDevice));

  kd_meta_args m;
  memset(&m, 0, sizeof m);
  m.B = B;
  m.T = T;
  m.D = D;
  m.mode = KD_MODE_CAUSAL;
  KD_OK_OR_FAIL(kd_plan_build(&m, plan, pbytes, NULL), "kd_plan_build");

  kd_attn_args a;
  memset(&a, 0, sizeof a);
  const int64_t st[3] = {(int64_t)H * T * D, (int64_t)T * D, D};
  a.q = dq_;
  a.k = dk_;
  a.v = dv_;
  a.o = o;
  a.dout = dd_;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  int64_t* strides[] = {a.q_strides, a.k_strides, a.v_strides, a.o_strides, a.do_strides,
                        a.dq_strides, a.dk_strides, a.dv_strides};
  for (int i = 0; i < 8; ++i) memcpy(strides[i], st, sizeof st);
  a.lse = dlse;
  a.delta = delta;
  a.o_lo = olo;
  a.B = B;
  a.H = H;
  a.T = T;
  a.D = D;
  a.dtype = KD_BF16;
  a.sm_scale = scale;
  a.precision = KD_PREC_SPLIT;
  /* a plan buffer smaller than the shape needs is refused before any launch */
  if (kd_attn_fwd(&a, plan, pbytes - 1, NULL) != KD_ERR_INVALID ||
      kd_attn_bwd(&a, plan, pbytes - 1, NULL) != KD_ERR_INVALID) {
    fprintf(stderr, "an undersized plan was not refused\n");
    return 1;
  }
  KD_OK_OR_FAIL(kd_attn_fwd(&a, plan, pbytes, NULL), "kd_attn_fwd");
  KD_OK_OR_FAIL(kd_attn_bwd(&a, plan, pbytes, NULL), "kd_attn_bwd");
  HIP_OK(hipDeviceSynchronize());
  void* outs[4] = {o, dq, dk, dv};
  for (int i = 0; i < 4; ++i) {
    HIP_OK(hipMemcpy(hbuf, outs[i], N * 2, hipMemcpyDeviceToHost));
    for (size_t j = 0; j < N; ++j) got[i][j] = from_bf16(hbuf[j]);
  }
  HIP_OK(hipMemcpy(lse, dlse, sizeof(float) * B * H * T, hipMemcpyDeviceToHost));

  int bad = check("bf16", x, x[0], x[1], got, lse);

  /* fp8 e4m3 scores: the per-(b, h) absmax of Q and of K, their e4m3 copies
   * and scales, then the same forward and backward reading q8 / k8 */
  uint8_t *q8, *k8;
  float *amax, *qsc, *ksc;
  HIP_OK(hipMalloc((void**)&q8, N));
  HIP_OK(hipMalloc((void**)&k8, N));
  HIP_OK(hipMalloc((void**)&amax, sizeof(float) * 2 * B * H));
  HIP_OK(hipMalloc((void**)&qsc, sizeof(float) * B * H));
  HIP_OK(hipMalloc((void**)&ksc, sizeof(float) * B * H));
  kd_quant_args qa;
  memset(&qa, 0, sizeof qa);
  memcpy(qa.x_strides, st, sizeof st);
  qa.B = B;
  qa.H = H;
  qa.T = T;
  qa.D = D;
  qa.dtype = KD_BF16;
  void* srcs[2] = {dq_, dk_};
  uint8_t* dsts[2] = {q8, k8};
  float* scales[2] = {qsc, ksc};
  for (int i = 0; i < 2; ++i) {
    qa.x = srcs[i];
    KD_OK_OR_FAIL(kd_absmax(&qa, amax + i * B * H, NULL), "kd_absmax");
    qa.amax = amax + i * B * H;
    qa.scale = scales[i];
    qa.y = dsts[i];
    KD_OK_OR_FAIL(kd_quant_fp8(&qa, NULL), "kd_quant_fp8");
  }
  a.q8 = q8;
  a.k8 = k8;
  a.q_scale = qsc;
  a.k_scale = ksc;
  KD_OK_OR_FAIL(kd_attn_fwd(&a, plan, pbytes, NULL), "kd_attn_fwd (fp8 scores)");
  KD_OK_OR_FAIL(kd_attn_bwd(&a, plan, pbytes, NULL), "kd_attn_bwd (fp8 scores)");
  HIP_OK(hipDeviceSynchronize());
  for (int i = 0; i < 4; ++i) {
    HIP_OK(hipMemcpy(hbuf, outs[i], N * 2, hipMemcpyDeviceToHost));
    for (size_t j = 0; j < N; ++j) got[i][j] = from_bf16(hbuf[j]);
  }
  HIP_OK(hipMemcpy(lse, dlse, sizeof(float) * B * H * T, hipMemcpyDeviceToHost));
  uint8_t* h8 = malloc(N);
  float hsc[B * H], *sq = malloc(N * sizeof(float)), *sk = malloc(N * sizeof(float));
  float* decoded[2] = {sq, sk};
  for (int i = 0; i < 2; ++i) {
    HIP_OK(hipMemcpy(h8, dsts[i], N, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(hsc, scales[i], sizeof hsc, hipMemcpyDeviceToHost));
    for (size_t j = 0; j < N; ++j) decoded[i][j] = from_e4m3(h8[j]) * hsc[j / ((size_t)T * D)];
  }
  bad |= check("fp8 scores", x, sq, sk, got, lse);
  printf(bad ? "c abi: MISMATCH\n" : "c abi ok\n");
  return bad;
}
