/*
 * megamoe_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Plain-C restatement of the integer/byte parts of the reference path, independent of the
 * torch/numpy restatement in megamoe_oracle.py so that the two can pin each other:
 *
 *  - oracle_e4m3_from_f32: float32 -> OCP FP8 E4M3 (e4m3fn: bias 7, no infinities, 0x7f/0xff
 *    NaN, max normal 448), round to nearest even, after the +-448 clip that the reference's
 *    quantising kernels apply first (megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:
 *    53-55, :121-142). Written from the OCP 8-bit floating point specification (v1.0).
 *  - oracle_route: the routing stage -- validity rule 0<=e<E && w!=0
 *    (deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:352), per-expert counts, tight
 *    exclusive-scan offsets (csrc/kernels/mega_moe_baseline_hip.cu:37-47), and the canonical
 *    stable order (ascending token*K+slot inside each expert) as a two-pass counting sort.
 *  - oracle_marlin_offset: deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66.
 *
 * Built by oracle/Makefile into oracle/liboracle.so.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint8_t oracle_e4m3_from_f32(float x) {
  if (isnan(x)) return 0x7f;
  uint8_t sign = signbit(x) ? 0x80 : 0x00;
  double a = fabs((double)x);
  if (a > 448.0) a = 448.0; /* the clip */
  if (a == 0.0) return sign;
  /* e4m3fn: normal exponents 1..15 (bias 7), subnormals 2^-6 * m/8, step 2^-9 */
  int e;
  frexp(a, &e);            /* a = f * 2^e, f in [0.5,1) -> a in [2^(e-1), 2^e) */
  int unbiased = e - 1;    /* a in [2^unbiased, 2^(unbiased+1)) */
  if (unbiased < -6) unbiased = -6; /* subnormal range shares the 2^-9 step */
  double step = ldexp(1.0, unbiased - 3);
  double q = a / step;     /* exact: power-of-two scaling */
  double fl = floor(q);
  double rem = q - fl;
  double n;
  if (rem > 0.5) n = fl + 1.0;
  else if (rem < 0.5) n = fl;
  else n = (fmod(fl, 2.0) == 0.0) ? fl : fl + 1.0;
  double v = n * step;     /* rounded magnitude */
  if (v > 448.0) v = 448.0;  /* cannot happen after the clip, kept for clarity */
  /* encode v */
  if (v < ldexp(1.0, -6)) {            /* subnormal: v = m * 2^-9, m in 0..7 */
    int m = (int)(v / ldexp(1.0, -9));
    return (uint8_t)(sign | (uint8_t)m);
  }
  int ev;
  double fv = frexp(v, &ev);           /* v = fv * 2^ev, fv in [0.5, 1) */
  int exp_field = ev - 1 + 7;          /* 1..15 */
  int mant = (int)((fv * 2.0 - 1.0) * 8.0 + 0.5);
  if (mant == 8) { mant = 0; exp_field += 1; }
  return (uint8_t)(sign | (uint8_t)(exp_field << 3) | (uint8_t)mant);
}

void oracle_e4m3_from_f32_array(uint8_t* out, const float* in, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_from_f32(in[i]);
}

float oracle_e4m3_to_f32(uint8_t b) {
  int sign = b & 0x80;
  int ex = (b >> 3) & 0xf;
  int m = b & 7;
  float v;
  if (ex == 0xf && m == 7) return NAN;
  if (ex == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, ex - 7);
  return sign ? -v : v;
}

int64_t oracle_marlin_offset(int e, int r, int k, int rows, int kdim) {
  const int64_t rt = r / 16, ri = r % 16, kt = k / 16, ki = k % 16;
  return (((int64_t)e * (rows / 16) + rt) * kdim + kt * 16) * 16 + ri * 16 + ki;
}

/* Two-pass counting sort. counts[E], offsets[E+1], output_index[S*K] (-1 if not routed),
 * row_token/row_slot/m_indices (int32 [R]), row_weight (f32 [R]). Returns R. */
int64_t oracle_route(const int64_t* topk_idx, const float* topk_w, int64_t num_tokens, int topk,
                     int num_experts, int32_t* counts, int32_t* offsets, int32_t* output_index,
                     int32_t* row_token, int32_t* row_slot, float* row_weight,
                     int32_t* m_indices) {
  const int64_t tasks = num_tokens * (int64_t)topk;
  memset(counts, 0, sizeof(int32_t) * (size_t)num_experts);
  for (int64_t t = 0; t < tasks; ++t) {
    const int64_t e = topk_idx[t];
    if (e >= 0 && e < num_experts && topk_w[t] != 0.0f) counts[e] += 1;
  }
  offsets[0] = 0;
  for (int e = 0; e < num_experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
  /* fill cursors */
  int32_t cursor_stack[4096];
  int32_t* cursor = cursor_stack;
  if (num_experts > 4096) return -1;
  for (int e = 0; e < num_experts; ++e) cursor[e] = offsets[e];
  for (int64_t t = 0; t < tasks; ++t) {
    const int64_t e = topk_idx[t];
    if (e >= 0 && e < num_experts && topk_w[t] != 0.0f) {
      const int32_t row = cursor[e]++;
      output_index[t] = row;
      row_token[row] = (int32_t)(t / topk);
      row_slot[row] = (int32_t)(t % topk);
      row_weight[row] = topk_w[t];
      m_indices[row] = (int32_t)e;
    } else {
      output_index[t] = -1;
    }
  }
  return offsets[num_experts];
}
