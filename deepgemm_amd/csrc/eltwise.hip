// eltwise.hip -- the HBM-bound stages around the GEMMs (gfx950):
//   * the top-k combine as an inverse-index gather (no atomics, fixed slot order):
//     y[t] = bf16(sum_s f32(part[output_index[t,s]])), the reference's reduce
//     (deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:706-760) and baseline gather
//     (csrc/kernels/mega_moe_baseline_hip.cu:98-127);
//   * row gather for the DeepEP-style preprocess, channelwise FP8 cast, Marlin pack.
#include "common.cuh"
#include "kernels.h"
#include "launch.h"

namespace mmoe {

namespace {

constexpr int kEltThreads = 256;
constexpr int kEltWaves = kEltThreads / kWave;

// ---------------------------------------------------------------- requant
// One wave per row: amax = max |y|; a = max(amax, 1e-4); act = e4m3(clip(y * (448/a)));
// act_scale = a/448 (the K2 requant, megamoe/dcu_megamoe_large_opt/K2_fused/
// k2_fused_ext.cu:341-364). A row of up to kRequantGroups*4*64 channels stays in registers
// between the reduction and the quantization; a longer one is read twice. y is GEMM1's SwiGLU
// x route weight output in bf16 (k2_fused_ext.cu:283-340, computed in GEMM1's epilogue and
// rounded as the reference's fused path rounds its activation, mega_moe_dcu_tiles.cuh:530-550).
constexpr int kRequantGroups = 8;  // float4 groups per lane held in registers

struct RequantArgs {
  const uint16_t* src;  // bf16 y [rows, I]
  float* amax;
  int32_t* meta;
  uint8_t* act;
  float* act_scale;
  int inter;
  RowDest dest;
  const int32_t* dual_rows;  // dual launches: the WIDE GEMM1 ran iff *dual_rows >= dual_min_rows
  int dual_min_rows;
};

// Nontemporal accesses for the streams these kernels touch once: y and the partial rows are
// read once, act is written once and read by GEMM2 from HBM anyway at prefill sizes. At c3 the
// requant went from 405 to 379 us and the combine from 427 to 410 us (same box, alternating
// builds); nontemporal stores of the combine's y rows were slower (436 us), so those stay plain.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4* p) {
  const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 ld_nt(const uint2* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// channels 4q .. 4q+3 of row `row`
__device__ __forceinline__ float4 requant_load(const RequantArgs& r, int64_t row, int q) {
  const uint2 b = ld_nt(reinterpret_cast<const uint2*>(r.src + row * r.inter) + q);
  return make_float4(bf16_to_f32(b.x & 0xffff), bf16_to_f32(b.x >> 16), bf16_to_f32(b.y & 0xffff),
                     bf16_to_f32(b.y >> 16));
}

// wide: the WIDE GEMM1 ran (meta[1]); direct: build the direct-write table
__device__ __forceinline__ void requant_rows(const RequantArgs& r, bool wide, bool direct) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int rows = r.meta[0];
  const int groups = r.inter >> 2;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    r.meta[1] = wide ? 1 : 0;
    if (r.dest.meta_flag != nullptr) *r.dest.meta_flag = direct ? 1 : 0;
  }
  for (int row = blockIdx.x * kEltWaves + wave; row < rows; row += gridDim.x * kEltWaves) {
    const int tok = direct ? r.dest.row_token[row] : 0;
    uint32_t* ar = reinterpret_cast<uint32_t*>(r.act + static_cast<int64_t>(row) * r.inter);
    float m = 0.0f;
    if ((r.inter & 7) == 0 && r.inter <= 8 * (kRequantGroups / 2) * kWave) {
      // 8 channels (16 bytes) a load, their 8 codes one 8-byte store
      const int octs = r.inter >> 3;
      const uint4* src = reinterpret_cast<const uint4*>(r.src + static_cast<int64_t>(row) * r.inter);
      float4 v[kRequantGroups];
#pragma unroll
      for (int j = 0; j < kRequantGroups / 2; ++j) {
        const int o = lane + j * kWave;
        const uint4 b = o < octs ? ld_nt(src + o) : make_uint4(0, 0, 0, 0);
        v[2 * j] = make_float4(bf16_to_f32(b.x & 0xffff), bf16_to_f32(b.x >> 16), bf16_to_f32(b.y & 0xffff),
                               bf16_to_f32(b.y >> 16));
        v[2 * j + 1] = make_float4(bf16_to_f32(b.z & 0xffff), bf16_to_f32(b.z >> 16), bf16_to_f32(b.w & 0xffff),
                                   bf16_to_f32(b.w >> 16));
        m = abs_max4(abs_max4(m, v[2 * j]), v[2 * j + 1]);
      }
      m = wave_max(m);
      const float inv = kE4m3Max / fmaxf(m, kAmaxFloor);
      u32x2_t* dst = reinterpret_cast<u32x2_t*>(r.act + static_cast<int64_t>(row) * r.inter);
#pragma unroll
      for (int j = 0; j < kRequantGroups / 2; ++j) {
        const int o = lane + j * kWave;
        const float4 a = v[2 * j], c = v[2 * j + 1];
        const u32x2_t codes = {pack_e4m3x4(a.x * inv, a.y * inv, a.z * inv, a.w * inv),
                               pack_e4m3x4(c.x * inv, c.y * inv, c.z * inv, c.w * inv)};
        if (o < octs) __builtin_nontemporal_store(codes, dst + o);
      }
    } else if (groups <= kRequantGroups * kWave) {
      float4 v[kRequantGroups];
#pragma unroll
      for (int i = 0; i < kRequantGroups; ++i) {
        const int q = lane + i * kWave;
        v[i] = q < groups ? requant_load(r, row, q) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        m = abs_max4(m, v[i]);
      }
      m = wave_max(m);
      const float inv = kE4m3Max / fmaxf(m, kAmaxFloor);
#pragma unroll
      for (int i = 0; i < kRequantGroups; ++i) {
        const int q = lane + i * kWave;
        if (q < groups) __builtin_nontemporal_store(pack_e4m3x4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv), ar + q);
      }
    } else {
      for (int q = lane; q < groups; q += kWave) m = abs_max4(m, requant_load(r, row, q));
      m = wave_max(m);
      const float inv = kE4m3Max / fmaxf(m, kAmaxFloor);
      for (int q = lane; q < groups; q += kWave) {
        const float4 v = requant_load(r, row, q);
        __builtin_nontemporal_store(pack_e4m3x4(v.x * inv, v.y * inv, v.z * inv, v.w * inv), ar + q);
      }
    }
    if (direct) {
      // the row's token has exactly one routed slot: GEMM2 writes its output row straight to y
      const int slot_row = lane < r.dest.topk
          ? r.dest.output_index[static_cast<int64_t>(tok) * r.dest.topk + lane] : -1;
      const int routed = __popcll(__ballot(slot_row >= 0));
      if (lane == 0) r.dest.row_dest[row] = routed == 1 ? tok : -1;
    }
    if (lane == 0) {
      r.amax[row] = m;
      r.act_scale[row] = fmaxf(m, kAmaxFloor) / kE4m3Max;
    }
  }
}

// kMode 0: after the 8-wave GEMM1, 1: after the WIDE GEMM1, 2: decided on the device (a dual
// GEMM1 launch; RequantArgs)
template <int kMode>
__global__ __launch_bounds__(kEltThreads) void requant_kernel(RequantArgs r) {
  // (after a dual launch the direct rows go with the WIDE GEMMs only)
  const bool wide = kMode == 1 || (kMode == 2 && *r.dual_rows >= r.dual_min_rows);
  const bool direct = r.dest.row_dest != nullptr && (kMode != 2 || wide);
  requant_rows(r, wide, direct);
}

// ---------------------------------------------------------------- combine
// One wave per (token, piece of V*64 16-byte column groups), grid-stride over those items; the
// next item's slot rows are loaded while the current one is summed, and the partial rows of up
// to 4 (V = 2) or 2 (V = 8) slots are loaded together. Lanes 0..K-1 hold the token's slot rows; every lane owns the 16-byte
// groups lane + 64j of the piece. Slots are summed in ascending order into fp32 accumulators
// that start at +0 (the reference's order); a token without routed slots gets zeros, and with
// skip_single a token with exactly one routed slot is left alone (GEMM2 wrote that row to y).
// V = 8 (whole 4096-column rows) for many tokens; V = 2 spreads few tokens over more waves.
template <int V>
__global__ __launch_bounds__(kEltThreads) void combine_kernel(CombineArgs c) {
  const int lane = lane_id();
  const int tokens = effective_tokens(c.runtime_tokens, c.host_tokens);
  const int nvec = c.hidden >> 3;
  const int parts = (nvec + kWave * V - 1) / (kWave * V);
  const int64_t items = static_cast<int64_t>(tokens) * parts;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEltWaves;
  int64_t it = static_cast<int64_t>(blockIdx.x) * kEltWaves + threadIdx.x / kWave;
  // lane < K: the row of slot `lane` of item i's token (-1: not routed) and its weight
  auto slot_row = [&](int64_t i, float& w) {
    w = 1.0f;
    if (i >= items || lane >= c.topk) return -1;
    const int64_t route = (i / parts) * c.topk + lane;
    int row = c.output_index[route];
    if (c.topk_ids != nullptr) {
      const int64_t ex = c.ids_i64 ? static_cast<const int64_t*>(c.topk_ids)[route]
                                   : static_cast<const int32_t*>(c.topk_ids)[route];
      if (ex < 0) row = -1;
    }
    if (c.apply_weights) w = c.topk_w[route];
    return row;
  };
  const bool skip_single = c.skip_single != nullptr && *c.skip_single != 0;
  // tokens below zdone without a routed slot: GEMM1 wrote their zero rows (ZeroFill)
  int64_t zdone = 0;
  if (c.zfill_claim != nullptr) {
    const int64_t claimed = *c.zfill_claim;
    const int64_t nchunks = (tokens + kZeroFillTokens - 1) / kZeroFillTokens;
    zdone = (claimed < nchunks ? claimed : nchunks) * kZeroFillTokens;
  }
  float w;
  int row = slot_row(it, w);
  for (; it < items; it += stride) {
    float next_w;
    const int next_row = slot_row(it + stride, next_w);
    const uint64_t routed = __ballot(row >= 0);
    if (!(skip_single && __popcll(routed) == 1) && !(routed == 0 && it / parts < zdone)) {
      const int64_t t = it / parts;
      const int v0 = static_cast<int>(it - t * parts) * kWave * V;
      float sum[V][8];
#pragma unroll
      for (int j = 0; j < V; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) sum[j][q] = 0.0f;
      // the routed slots in ascending order, kSlots at a time: their rows' loads go out together
      // (one round trip per batch instead of one per slot), the sums stay in slot order
      constexpr int kSlots = V <= 2 ? 4 : 2;
      for (uint64_t m = routed; m != 0;) {
        uint4 p[kSlots][V];
        float ws[kSlots];
        bool has[kSlots];
#pragma unroll
        for (int b = 0; b < kSlots; ++b) {
          has[b] = m != 0;  // wave-uniform (a ballot)
          const int s = has[b] ? __ffsll(static_cast<unsigned long long>(m)) - 1 : 0;
          m &= m - 1;
          const int r = __shfl(row, s, kWave);
          ws[b] = __shfl(w, s, kWave);
          const uint4* prow = reinterpret_cast<const uint4*>(c.part + static_cast<int64_t>(r) * c.hidden);
#pragma unroll
          for (int j = 0; j < V; ++j) {
            const int v = v0 + j * kWave + lane;
            p[b][j] = has[b] && v < nvec ? ld_nt(prow + v) : make_uint4(0, 0, 0, 0);
          }
        }
#pragma unroll
        for (int b = 0; b < kSlots; ++b) {
          if (!has[b]) break;
#pragma unroll
          for (int j = 0; j < V; ++j) {
            const uint32_t words[4] = {p[b][j].x, p[b][j].y, p[b][j].z, p[b][j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float lo = bf16_to_f32(words[q] & 0xffff);
              float hi = bf16_to_f32(words[q] >> 16);
              if (c.apply_weights) { lo *= ws[b]; hi *= ws[b]; }
              sum[j][2 * q] += lo;
              sum[j][2 * q + 1] += hi;
            }
          }
        }
      }
      uint4* yrow = reinterpret_cast<uint4*>(c.y + t * c.hidden);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int v = v0 + j * kWave + lane;
        if (v < nvec)
          yrow[v] = make_uint4(pack_bf16x2(sum[j][0], sum[j][1]), pack_bf16x2(sum[j][2], sum[j][3]),
                               pack_bf16x2(sum[j][4], sum[j][5]), pack_bf16x2(sum[j][6], sum[j][7]));
      }
    }
    row = next_row;
    w = next_w;
  }
}

// Scalar tail of the combine for hidden % 8 != 0 (kept simple; the layer uses H % 128 == 0).
__global__ __launch_bounds__(kEltThreads) void combine_scalar_kernel(CombineArgs c) {
  const int tokens = effective_tokens(c.runtime_tokens, c.host_tokens);
  for (int t = blockIdx.x; t < tokens; t += gridDim.x) {
    for (int h = threadIdx.x; h < c.hidden; h += kEltThreads) {
      float sum = 0.0f;
      for (int s = 0; s < c.topk; ++s) {
        const int64_t route = static_cast<int64_t>(t) * c.topk + s;
        const int row = c.output_index[route];
        if (row < 0) continue;
        if (c.topk_ids != nullptr) {
          const int64_t ex = c.ids_i64 ? static_cast<const int64_t*>(c.topk_ids)[route]
                                       : static_cast<const int32_t*>(c.topk_ids)[route];
          if (ex < 0) continue;
        }
        float v = bf16_to_f32(c.part[static_cast<int64_t>(row) * c.hidden + h]);
        if (c.apply_weights) v *= c.topk_w[route];
        sum += v;
      }
      c.y[static_cast<int64_t>(t) * c.hidden + h] = f32_to_bf16(sum);
    }
  }
}

// ---------------------------------------------------------------- task gather (preprocess)
__global__ __launch_bounds__(kEltThreads) void gather_tasks_kernel(uint8_t* gx, float* gs,
                                                                   const uint8_t* x,
                                                                   const float* x_sf,
                                                                   const int32_t* output_index,
                                                                   int64_t tasks, int topk,
                                                                   int hidden) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  for (int64_t task = static_cast<int64_t>(blockIdx.x) * kEltWaves + wave; task < tasks;
       task += static_cast<int64_t>(gridDim.x) * kEltWaves) {
    const int64_t r = output_index[task];
    if (r < 0) continue;
    const int64_t tok = task / topk;
    const uint8_t* src = x + static_cast<int64_t>(tok) * hidden;
    uint8_t* dst = gx + r * hidden;
    if ((hidden & 15) == 0) {
      for (int v = lane; v < (hidden >> 4); v += kWave)
        reinterpret_cast<uint4*>(dst)[v] = reinterpret_cast<const uint4*>(src)[v];
    } else {
      for (int v = lane; v < hidden; v += kWave) dst[v] = src[v];
    }
    if (lane == 0) gs[r] = x_sf[tok];
  }
}

// ---------------------------------------------------------------- channelwise cast
__global__ __launch_bounds__(kEltThreads) void cast_fp8_rows_kernel(uint8_t* out, float* scale,
                                                                    const uint16_t* x,
                                                                    int64_t rows, int64_t cols) {
  __shared__ float s_red[kEltWaves];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint16_t* xr = x + r * cols;
    float amax = 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += kEltThreads) amax = fmaxf(amax, fabsf(bf16_to_f32(xr[c])));
    amax = wave_max(amax);
    if (lane_id() == 0) s_red[threadIdx.x / kWave] = amax;
    __syncthreads();
    float m = s_red[0];
    for (int w = 1; w < kEltWaves; ++w) m = fmaxf(m, s_red[w]);
    const float sc = fmaxf(m, kAmaxFloor) / kE4m3Max;
    if (threadIdx.x == 0) scale[r] = sc;
    uint8_t* orow = out + r * cols;
    for (int64_t c = threadIdx.x; c < cols; c += kEltThreads) orow[c] = f32_to_e4m3(bf16_to_f32(xr[c]) / sc);
    __syncthreads();
  }
}

// ---------------------------------------------------------------- Marlin pack
// out[g, r/16, (k/16)*256 + (r%16)*16 + k%16] = in[g, r, k]; one thread per 16-byte block row.
__global__ __launch_bounds__(kEltThreads) void marlin_pack_kernel(uint8_t* out, const uint8_t* in,
                                                                  int64_t groups, int64_t rows,
                                                                  int64_t k) {
  const int64_t kblocks = k >> 4;
  const int64_t total = groups * rows * kblocks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEltThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kEltThreads) {
    const int64_t kb = i % kblocks;
    const int64_t gr = i / kblocks;  // g * rows + r
    const int64_t r = gr % rows;
    const int64_t gidx = gr / rows;
    const uint4 v = *reinterpret_cast<const uint4*>(in + gr * k + kb * 16);
    const int64_t dst = ((gidx * (rows >> 4) + (r >> 4)) * k + kb * 16) * 16 + (r & 15) * 16;
    *reinterpret_cast<uint4*>(out + dst) = v;
  }
}

__global__ __launch_bounds__(kEltThreads) void f32_to_e4m3_kernel(uint8_t* out, const float* in,
                                                                  int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEltThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kEltThreads)
    out[i] = f32_to_e4m3(in[i]);
}

unsigned grid_for(int64_t work_items, int64_t per_block, int64_t cap) {
  int64_t g = (work_items + per_block - 1) / per_block;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace

hipError_t launch_requant(const uint16_t* src, bool wide, float* amax, int32_t* meta, uint8_t* act,
                          float* act_scale, int64_t max_rows, int inter, const RowDest& dest,
                          int num_cus, hipStream_t stream, const int32_t* dual_rows,
                          int dual_min_rows) {
  if (max_rows <= 0) return hipSuccess;
  if (inter % 4) return hipErrorInvalidValue;
  if (dest.row_dest != nullptr && (dest.row_token == nullptr || dest.output_index == nullptr ||
                                   dest.topk < 1 || dest.topk > kWave))
    return hipErrorInvalidValue;
  const RequantArgs r{src, amax, meta, act, act_scale, inter, dest, dual_rows, dual_min_rows};
  // grid of up to 16 workgroups a CU (one row per wave in flight; the hardware keeps what fits
  // resident): 397 us at 195,558 rows vs 470 us with 4 a CU
  const unsigned grid = grid_for(max_rows, kEltWaves, static_cast<int64_t>(num_cus) * 16);
  if (dual_rows != nullptr)
    return launch_kernel(requant_kernel<2>, dim3(grid), dim3(kEltThreads), 0, stream, r);
  if (wide) return launch_kernel(requant_kernel<1>, dim3(grid), dim3(kEltThreads), 0, stream, r);
  return launch_kernel(requant_kernel<0>, dim3(grid), dim3(kEltThreads), 0, stream, r);
}

hipError_t launch_combine(const CombineArgs& c, int num_cus, hipStream_t stream) {
  if (c.host_tokens <= 0) return hipSuccess;
  if (c.topk > 16) return hipErrorInvalidValue;
  if ((c.hidden & 7) == 0) {
    // a wave per item, up to 8 four-wave workgroups a CU in flight; whole rows once there are
    // at least 16 tokens a CU
    const int64_t nvec = c.hidden >> 3;
    if (c.host_tokens >= static_cast<int64_t>(num_cus) * 16) {
      const int64_t items = c.host_tokens * ((nvec + kWave * 8 - 1) / (kWave * 8));
      const unsigned grid = grid_for(items, kEltWaves, static_cast<int64_t>(num_cus) * 8);
      return launch_kernel(combine_kernel<8>, dim3(grid), dim3(kEltThreads), 0, stream, c);
    } else {
      const int64_t items = c.host_tokens * ((nvec + kWave * 2 - 1) / (kWave * 2));
      const unsigned grid = grid_for(items, kEltWaves, static_cast<int64_t>(num_cus) * 8);
      return launch_kernel(combine_kernel<2>, dim3(grid), dim3(kEltThreads), 0, stream, c);
    }
  } else {
    if (c.skip_single != nullptr) return hipErrorInvalidValue;
    const unsigned grid = grid_for(c.host_tokens, 1, static_cast<int64_t>(num_cus) * 16);
    return launch_kernel(combine_scalar_kernel, dim3(grid), dim3(kEltThreads), 0, stream, c);
  }
}

hipError_t launch_gather_tasks(uint8_t* grouped_x, float* grouped_scale, const uint8_t* x,
                               const float* x_sf, const int32_t* output_index, int64_t tasks,
                               int topk, int hidden, hipStream_t stream) {
  if (tasks <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_tasks_kernel, dim3(grid_for(tasks, kEltWaves, 8192)),
                     dim3(kEltThreads), 0, stream, grouped_x, grouped_scale, x, x_sf,
                     output_index, tasks, topk, hidden);
  return hipGetLastError();
}

hipError_t launch_cast_fp8_channelwise(uint8_t* out, float* scale, const uint16_t* x,
                                       int64_t rows, int64_t cols, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(cast_fp8_rows_kernel, dim3(grid_for(rows, 1, 65536)), dim3(kEltThreads), 0,
                     stream, out, scale, x, rows, cols);
  return hipGetLastError();
}

hipError_t launch_marlin_pack(uint8_t* out, const uint8_t* in, int64_t groups, int64_t rows,
                              int64_t k, hipStream_t stream) {
  const int64_t total = groups * rows * (k >> 4);
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(marlin_pack_kernel, dim3(grid_for(total, kEltThreads, 65536)),
                     dim3(kEltThreads), 0, stream, out, in, groups, rows, k);
  return hipGetLastError();
}

hipError_t launch_f32_to_e4m3(uint8_t* out, const float* in, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(f32_to_e4m3_kernel, dim3(grid_for(n, kEltThreads, 65536)), dim3(kEltThreads),
                     0, stream, out, in, n);
  return hipGetLastError();
}

}  // namespace mmoe
