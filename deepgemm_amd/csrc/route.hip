// route.hip -- deterministic routing for the grouped expert GEMMs (gfx950).
//
// Semantics (reference): a task (token t, slot s) is routed to local expert e =
// topk_idx[t,s] iff 0 <= e < E and, for the layer, topk_weights[t,s] != 0
// (deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:352). Routed rows are
// expert-contiguous at tight exclusive-scan offsets (csrc/kernels/mega_moe_baseline_hip.cu:
// 37-47). The reference places rows inside an expert by atomicAdd arrival
// (mega_moe_baseline_hip.cu:75, mega_moe_dcu.cuh:359); here the order is the stable one --
// ascending task index -- so counts, rows and output_index are bitwise reproducible.
//
// Three launches, all O(S*K) integer work, HBM-bound on the topk tables:
//   1. count:   one workgroup per chunk of 1024 tasks, LDS histogram -> chunk_counts[c][e]
//   2. scan:    one workgroup; per expert, exclusive scan over chunks (wave prefix sums),
//               expert offsets, R, stats += counts
//   3. scatter: one workgroup per chunk; stable rank of each task among equal experts via
//               wave ballot/popcount (a match loop over the distinct experts of the wave)
//               plus per-wave bases in LDS; writes output_index and the per-row tables.
#include "common.cuh"
#include "kernels.h"

namespace mmoe {

namespace {

constexpr int kRouteThreads = 256;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kTasksPerWave = kRouteChunk / kRouteWaves;  // 256 contiguous tasks per wave
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int task_expert(const RouteArgs& a, int64_t task) {
  int64_t e = a.idx_i64 ? static_cast<const int64_t*>(a.topk_idx)[task]
                        : static_cast<int64_t>(static_cast<const int32_t*>(a.topk_idx)[task]);
  if (e < 0 || e >= a.num_experts) return -1;
  if (a.check_weight && a.topk_w[task] == 0.0f) return -1;
  return static_cast<int>(e);
}

__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(RouteArgs a) {
  __shared__ int s_cnt[kMaxExperts];
  const int tid = threadIdx.x;
  for (int e = tid; e < a.num_experts; e += kRouteThreads) s_cnt[e] = 0;
  __syncthreads();
  const int64_t ntasks = static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kRouteChunk;
  for (int i = tid; i < kRouteChunk; i += kRouteThreads) {
    const int64_t task = base + i;
    if (task < ntasks) {
      const int e = task_expert(a, task);
      if (e >= 0) atomicAdd(&s_cnt[e], 1);
    }
  }
  __syncthreads();
  int32_t* dst = a.chunk_counts + static_cast<int64_t>(blockIdx.x) * a.num_experts;
  for (int e = tid; e < a.num_experts; e += kRouteThreads) dst[e] = s_cnt[e];
}

__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_up(v, off, kWave);
    if (lane >= off) v += u;
  }
  return v;
}

__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(RouteArgs a, int num_chunks) {
  __shared__ int s_tot[kMaxExperts];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  constexpr int waves = kScanThreads / kWave;
  for (int e = wave; e < a.num_experts; e += waves) {
    int carry = 0;
    for (int c0 = 0; c0 < num_chunks; c0 += kWave) {
      const int c = c0 + lane;
      int32_t* p = a.chunk_counts + static_cast<int64_t>(c) * a.num_experts + e;
      const int v = c < num_chunks ? *p : 0;
      const int inc = wave_inclusive_scan(v);
      if (c < num_chunks) *p = carry + inc - v;  // exclusive base of chunk c for expert e
      carry += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) s_tot[e] = carry;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t off = 0;
    for (int e = 0; e < a.num_experts; ++e) {
      a.offsets[e] = static_cast<int32_t>(off);
      off += a.given_counts != nullptr ? a.given_counts[e] : s_tot[e];
    }
    a.offsets[a.num_experts] = static_cast<int32_t>(off);
    int64_t routed = 0;
    for (int e = 0; e < a.num_experts; ++e) routed += s_tot[e];
    a.meta[0] = static_cast<int32_t>(routed < a.row_cap ? routed : a.row_cap);
  }
  for (int e = threadIdx.x; e < a.num_experts; e += kScanThreads) {
    a.counts[e] = s_tot[e];
    if (a.stats != nullptr) a.stats[e] += s_tot[e];
  }
}

__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(RouteArgs a) {
  __shared__ int s_wbase[kRouteWaves][kMaxExperts];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int64_t ntasks = static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk;
  const int64_t chunk_base = static_cast<int64_t>(blockIdx.x) * kRouteChunk;
  const int64_t wave_base = chunk_base + static_cast<int64_t>(wave) * kTasksPerWave;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));

  // pass 1: per-wave counts per expert
  for (int e = tid; e < kRouteWaves * a.num_experts; e += kRouteThreads)
    s_wbase[e / a.num_experts][e % a.num_experts] = 0;
  __syncthreads();
  for (int p = 0; p < kTasksPerWave; p += kWave) {
    const int64_t task = wave_base + p + lane;
    const int e = task < ntasks ? task_expert(a, task) : -1;
    uint64_t active = __ballot(e >= 0);
    while (active != 0ull) {
      const int leader = __ffsll(static_cast<unsigned long long>(active)) - 1;
      const int le = __shfl(e, leader, kWave);
      const uint64_t m = __ballot(e == le);
      if (lane == leader) s_wbase[wave][le] += __popcll(m);
      active &= ~m;
    }
  }
  __syncthreads();
  // per-wave bases: expert offset + chunk base + counts of the earlier waves of this chunk
  const int32_t* cbase = a.chunk_counts + static_cast<int64_t>(blockIdx.x) * a.num_experts;
  for (int e = tid; e < a.num_experts; e += kRouteThreads) {
    int run = a.offsets[e] + cbase[e];
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = s_wbase[w][e];
      s_wbase[w][e] = run;
      run += c;
    }
  }
  __syncthreads();
  // pass 2: stable ranks -> rows
  for (int p = 0; p < kTasksPerWave; p += kWave) {
    const int64_t task = wave_base + p + lane;
    const bool in_range = task < ntasks;
    const int e = in_range ? task_expert(a, task) : -1;
    int row = -1;
    uint64_t active = __ballot(e >= 0);
    while (active != 0ull) {
      const int leader = __ffsll(static_cast<unsigned long long>(active)) - 1;
      const int le = __shfl(e, leader, kWave);
      const uint64_t m = __ballot(e == le);
      const int base = s_wbase[wave][le];
      if (e == le) row = base + __popcll(m & lt_mask);
      __builtin_amdgcn_wave_barrier();
      if (lane == leader) s_wbase[wave][le] = base + __popcll(m);
      __builtin_amdgcn_wave_barrier();
      active &= ~m;
    }
    if (row >= 0 && row >= a.row_cap) row = -1;
    if (in_range) a.output_index[task] = row;
    if (row >= 0) {
      a.row_token[row] = static_cast<int32_t>(task / a.topk);
      if (a.row_weight != nullptr) a.row_weight[row] = a.topk_w[task];
      if (a.m_indices != nullptr) a.m_indices[row] = e;
    }
  }
}

}  // namespace

hipError_t launch_route(const RouteArgs& a, int64_t num_chunks, hipStream_t stream) {
  if (num_chunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(route_count_kernel, dim3(static_cast<unsigned>(num_chunks)), dim3(kRouteThreads),
                     0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a,
                     static_cast<int>(num_chunks));
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(route_scatter_kernel, dim3(static_cast<unsigned>(num_chunks)),
                     dim3(kRouteThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mmoe
