// common.cuh -- gfx950 device helpers shared by the Mega MoE kernels.
//
// Number formats: OCP FP8 E4M3 (e4m3fn, the bytes of torch.float8_e4m3fn) for activations
// and weights; bf16 with round-to-nearest-even for the GEMM outputs and the layer output.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmoe {

constexpr float kE4m3Max = 448.0f;
constexpr float kAmaxFloor = 1.0e-4f;
constexpr int kWave = 64;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 by the gfx950 conversion instruction (v_cvt_pk_bf16_f32:
// two values per instruction). Finite inputs only matter: the layer never produces NaN/Inf
// from finite FP8 operands and finite scales.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pack_bf16x2(f, 0.0f) & 0xffffu);
}

// SwiGLU x route weight of one channel from the bf16-rounded gate g and up u: the clamp of the
// staged K2 (u to [-c, c], g to <= c), then g * sigmoid(g) * u * w left to right with the
// fast-math sigmoid of the reference's fused path (hardware exp2 and reciprocal:
// deep_gemm/include/deep_gemm/common/mega_moe_dcu.cuh:89-98; the staged K2 uses __expf,
// megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:328).
// kClamp fixed at compile time: without a clamp the compiler emits none of its instructions
// (chosen per element at run time, it had computed the clamp for every channel and selected).
template <bool kClamp>
__device__ __forceinline__ float swiglu_weighted_c(float g, float u, float w, float c) {
  if constexpr (kClamp) {
    u = fminf(c, fmaxf(-c, u));
    g = fminf(c, g);
  }
  constexpr float kLog2E = 1.4426950408889634f;
  const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2E));
  return g * sig * u * w;
}

__device__ __forceinline__ float swiglu_weighted(float g, float u, float w, bool has_clamp, float c) {
  return has_clamp ? swiglu_weighted_c<true>(g, u, w, c) : swiglu_weighted_c<false>(g, u, w, c);
}

__device__ __forceinline__ float clip_e4m3(float v) {
  return fminf(kE4m3Max, fmaxf(-kE4m3Max, v));
}

// Four floats -> four e4m3fn bytes (little-endian in one u32). Clip to +-448 first, then the
// gfx950 hardware conversion (round to nearest even, OCP encoding).
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(clip_e4m3(a), clip_e4m3(b), 0, false);
  p = __builtin_amdgcn_cvt_pk_fp8_f32(clip_e4m3(c), clip_e4m3(d), p, true);
  return static_cast<uint32_t>(p);
}

__device__ __forceinline__ uint8_t f32_to_e4m3(float a) {
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(clip_e4m3(a), 0.0f, 0, false);
  return static_cast<uint8_t>(p & 0xff);
}

__device__ __forceinline__ float abs_max4(float m, const float4& v) {
  return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
  return v;
}

// Max of v >= 0 over each half-wave (lanes 0-31, 32-63), valid in lanes 16-31 and 48-63 (all
// lanes active), by DPP: quad swaps, half-row and row mirrors give every lane its 16-lane row's
// max, then row_bcast:15 brings row 0's max into row 1 and row 2's into row 3 (other rows: 0).
template <int kCtrl, int kRows>
__device__ __forceinline__ float dpp_max_step(float x) {
  return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, kRows, 0xf, false)));
}

__device__ __forceinline__ float half_wave_max_nonneg(float v) {
  v = dpp_max_step<0xb1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_max_step<0x4e, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_max_step<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_max_step<0x140, 0xf>(v);  // row_mirror
  return dpp_max_step<0x142, 0xa>(v);  // row_bcast:15, rows 1 and 3
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active), by DPP: row shifts 1, 2,
// 4, 8 within each 16-lane row (a lane without a source adds 0), then row 0's total into row 1
// and row 2's into row 3 (row_bcast:15), then rows 0-1's total into rows 2 and 3 (row_bcast:31).
// Six dependent VALU steps, no LDS permutes.
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
  return v;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Number of tokens this call processes: the device scalar (clamped to [0, cap]) when given,
// else the host value.
__device__ __forceinline__ int effective_tokens(const int32_t* runtime_tokens, int host_tokens) {
  if (runtime_tokens == nullptr) return host_tokens;
  int v = *runtime_tokens;
  return v < 0 ? 0 : (v > host_tokens ? host_tokens : v);
}

}  // namespace mmoe
