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
// Ranks come from wave ballots: one ballot per bit of the expert id gives every lane the mask
// of lanes holding the same expert (a match-any in log2(E) votes); a lane's rank is the
// popcount of that mask below it and the group's lowest lane publishes the group size. Per-wave
// counts become per-wave bases through LDS prefix sums.
//
// Two launch shapes, both integer work bound by the topk tables' HBM reads:
//   * small (<= 16384 tasks): ONE workgroup of 16 waves does count, scan and scatter;
//   * large: a count kernel (one workgroup per chunk, LDS histogram) and a scatter kernel
//     (one workgroup per chunk) that rebuilds the expert offsets and its chunk base from the
//     per-chunk counts itself, so no grid-wide barrier or separate scan launch is needed.
#include "launch.h"
#include "route_wave.cuh"

namespace mmoe {

namespace {

constexpr int kSmallThreads = 1024;
constexpr int kSmallWaves = kSmallThreads / kWave;
constexpr int kSmallMaxExperts = 256;
constexpr int kChunkThreads = 1024;
constexpr int kChunkWaves = kChunkThreads / kWave;
static_assert(kMaxExperts <= kChunkThreads, "the chunk-count reduction needs a thread per expert");
static_assert(2 * kChunkThreads <= kChunkWaves * kMaxExperts, "partial sums fit in s_wbase");
static_assert(kChunkWaves == kRouteWaves, "per-wave counts of a chunk in the workspace");

// Assigns rows to one 64-task pass in task order; base[e] is this wave's running base.
__device__ __forceinline__ void wave_scatter_pass(const RouteArgs& a, int64_t task, bool in_range,
                                                  int e, float w, int id_bits, int* base) {
  const uint64_t m = match_expert(e, id_bits);
  int row = -1;
  if (e >= 0) row = base[e] + __popcll(m & lanes_below());
  __builtin_amdgcn_wave_barrier();
  if (e >= 0 && (m & lanes_below()) == 0ull) base[e] += __popcll(m);
  __builtin_amdgcn_wave_barrier();
  if (row >= 0 && row >= a.row_cap) row = -1;
  if (in_range) a.output_index[task] = row;
  if (row >= 0) {
    a.row_token[row] = static_cast<int32_t>(task / a.topk);
    if (a.row_weight != nullptr) a.row_weight[row] = w;
    if (a.m_indices != nullptr) a.m_indices[row] = e;
  }
}

// Counts then scatters the tasks [begin, end) of this wave, in batches of kBatch passes held
// in registers. `cnt` is the wave's count row (zeroed by the caller); between the two phases
// the caller turns counts into bases (needs a workgroup barrier), passed through `phase_gap`.
constexpr int kBatch = 8;

// Counts of the tasks [begin, end) of this wave into its count row.
__device__ void wave_count_range(const RouteArgs& a, int64_t begin, int64_t end, int* row) {
  int ev[kBatch];
  float wv[kBatch];
  const int id_bits = expert_id_bits(a.num_experts);
  for (int64_t b = begin; b < end; b += kBatch * kWave) {
    wave_load<kBatch>(a, b, end, ev, wv);
#pragma unroll
    for (int p = 0; p < kBatch; ++p) wave_count_pass(ev[p], id_bits, row);
  }
}

// counted: the count rows hold this range's counts already (the count kernel's).
template <class Gap>
__device__ void wave_route(const RouteArgs& a, int64_t begin, int64_t end, int* row,
                           Gap phase_gap, bool counted = false) {
  int ev[kBatch];
  float wv[kBatch];
  const int id_bits = expert_id_bits(a.num_experts);
  if (!counted) wave_count_range(a, begin, end, row);
  phase_gap();
  const int lane = lane_id();
  for (int64_t b = begin; b < end; b += kBatch * kWave) {
    wave_load<kBatch>(a, b, end, ev, wv);
#pragma unroll
    for (int p = 0; p < kBatch; ++p) {
      const int64_t task = b + p * kWave + lane;
      wave_scatter_pass(a, task, task < end, ev[p], wv[p], id_bits, row);
    }
  }
}

// Expert offsets from totals (exclusive scan, or the caller's counts for the preprocess), by
// wave 0 in 64-expert chunks (DPP scans); fills s_off[0..E], and the writer workgroup
// publishes offsets, counts, stats, the routed row count (meta[0]) and the largest expert's
// row count (meta[4]).
__device__ void publish_offsets(const RouteArgs& a, const int* s_tot, int* s_off, bool writer) {
  if (threadIdx.x < kWave) {
    const int lane = lane_id();
    int carry = 0, routed = 0, largest = 0;
    for (int e0 = 0; e0 < a.num_experts; e0 += kWave) {
      const int e = e0 + lane;
      const int tot = e < a.num_experts ? s_tot[e] : 0;
      const int c = a.given_counts != nullptr ? (e < a.num_experts ? a.given_counts[e] : 0) : tot;
      const int inc = wave_inclusive_sum(c);
      if (e < a.num_experts) s_off[e] = carry + inc - c;
      carry += __shfl(inc, kWave - 1, kWave);
      routed += __shfl(wave_inclusive_sum(tot), kWave - 1, kWave);
      largest = max(largest, wave_max(tot));
    }
    if (lane == 0) {
      s_off[a.num_experts] = carry;
      if (writer) {
        a.meta[0] = static_cast<int32_t>(routed < a.row_cap ? routed : a.row_cap);
        a.meta[3] = 0;  // the call's status: the staged kernels have no bounded waits
        a.meta[4] = largest;
      }
    }
  }
  __syncthreads();
  if (writer) {
    for (int e = threadIdx.x; e <= a.num_experts; e += blockDim.x) a.offsets[e] = s_off[e];
    for (int e = threadIdx.x; e < a.num_experts; e += blockDim.x) {
      a.counts[e] = s_tot[e];
      if (a.stats != nullptr) a.stats[e] += s_tot[e];
    }
  }
}

// A routing launch that GEMM1 stands in for (the live tasks fit its in-kernel routing).
__device__ __forceinline__ bool route_skipped(const RouteArgs& a) {
  return a.fused_max_tasks > 0 &&
         static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk <= a.fused_max_tasks;
}

// The routing launch runs before the GEMMs of a layer: it zeroes their claim counters.
__device__ __forceinline__ void zero_sched(const RouteArgs& a) {
  if (blockIdx.x == 0 && a.zero_ints != nullptr)
    for (int i = threadIdx.x; i < a.zero_count; i += blockDim.x) a.zero_ints[i] = 0;
}

__global__ __launch_bounds__(kSmallThreads) void route_small_kernel(RouteArgs a) {
  zero_sched(a);  // (also when GEMM1 routes: the WIDE GEMM1 then returns at once, and the
                  // combine reads its zero-fill claim counter as zero)
  if (route_skipped(a)) return;
  __shared__ int s_cnt[kSmallWaves][kSmallMaxExperts];
  __shared__ int s_tot[kSmallMaxExperts];
  __shared__ int s_off[kSmallMaxExperts + 1];
  const int wave = threadIdx.x / kWave;
  const int E = a.num_experts;
  const int64_t ntasks =
      static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk;
  const int64_t per = ((ntasks + kSmallWaves - 1) / kSmallWaves + kWave - 1) / kWave * kWave;
  const int64_t begin = wave * per;
  const int64_t end = begin + per < ntasks ? begin + per : ntasks;
  for (int i = threadIdx.x; i < kSmallWaves * E; i += kSmallThreads) s_cnt[i / E][i % E] = 0;
  __syncthreads();
  wave_route(a, begin, end, s_cnt[wave], [&]() {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kSmallThreads) {
      int run = 0;
      for (int w = 0; w < kSmallWaves; ++w) {
        const int c = s_cnt[w][e];
        s_cnt[w][e] = run;
        run += c;
      }
      s_tot[e] = run;
    }
    __syncthreads();
    publish_offsets(a, s_tot, s_off, true);
    for (int i = threadIdx.x; i < kSmallWaves * E; i += kSmallThreads) s_cnt[i / E][i % E] += s_off[i % E];
    __syncthreads();
  });
}

// The tasks of chunk `chunk` that wave `wave` of a chunk workgroup routes: the same split in
// the count and the scatter kernels, so the scatter can take the count kernel's per-wave counts.
struct WaveRange {
  int64_t begin, end;
};
__device__ __forceinline__ WaveRange chunk_wave_range(int64_t ntasks, int chunk, int chunk_tasks, int wave) {
  const int64_t cbegin = static_cast<int64_t>(chunk) * chunk_tasks;
  const int64_t cend = cbegin + chunk_tasks < ntasks ? cbegin + chunk_tasks : ntasks;
  const int64_t per = ((chunk_tasks / kChunkWaves) + kWave - 1) / kWave * kWave;
  const int64_t begin = cbegin + wave * per < cend ? cbegin + wave * per : cend;
  return WaveRange{begin, begin + per < cend ? begin + per : cend};
}

// Per-wave counts of a chunk (each wave's ballot counts of its own task range, no atomics);
// writes the chunk's totals and, when wave_counts is given, the per-wave rows.
__global__ __launch_bounds__(kChunkThreads) void route_count_kernel(RouteArgs a, int chunk_tasks) {
  __shared__ int s_cnt[kChunkWaves][kMaxExperts];
  zero_sched(a);
  if (route_skipped(a)) return;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int E = a.num_experts;
  for (int i = tid; i < kChunkWaves * E; i += kChunkThreads) s_cnt[i / E][i % E] = 0;
  __syncthreads();
  const int64_t ntasks =
      static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk;
  const WaveRange wr = chunk_wave_range(ntasks, blockIdx.x, chunk_tasks, wave);
  wave_count_range(a, wr.begin, wr.end, s_cnt[wave]);
  __syncthreads();
  int32_t* dst = a.chunk_counts + static_cast<int64_t>(blockIdx.x) * E;
  for (int e = tid; e < E; e += kChunkThreads) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kChunkWaves; ++w) tot += s_cnt[w][e];
    dst[e] = tot;
  }
  if (a.wave_counts != nullptr) {
    int32_t* wdst = a.wave_counts + static_cast<int64_t>(blockIdx.x) * kChunkWaves * E;
    for (int i = tid; i < kChunkWaves * E; i += kChunkThreads) wdst[i] = s_cnt[i / E][i % E];
  }
}


__global__ __launch_bounds__(kChunkThreads) void route_chunk_scatter_kernel(RouteArgs a,
                                                                            int chunk_tasks,
                                                                            int num_chunks) {
  if (route_skipped(a)) return;
  __shared__ int s_wbase[kChunkWaves][kMaxExperts];
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_cbase[kMaxExperts];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int E = a.num_experts;
  const int chunk = blockIdx.x;
  // Totals and this chunk's base per expert, from every chunk's counts. Thread t sums the
  // chunks g, g + G, g + 2G, ... of expert e = t % E (g = t / E, G = 1024 / E groups), so all
  // threads load at once (consecutive threads, consecutive experts of a chunk row); the G
  // partial sums of an expert then meet in LDS (s_wbase as scratch, before its own use).
  {
    const int groups = kChunkThreads / E;  // >= 1: E <= kMaxExperts == kChunkThreads
    int* s_ptot = &s_wbase[0][0];
    int* s_pbase = s_ptot + groups * E;   // 2 * groups * E <= 2 * 1024 ints of s_wbase
    if (tid < groups * E) {
      const int e = tid % E, g = tid / E;
      int tot = 0, base = 0;
      int c = g;
      for (; c + 7 * groups < num_chunks; c += 8 * groups) {  // 8 loads in flight together
        int v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = a.chunk_counts[static_cast<int64_t>(c + j * groups) * E + e];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          tot += v[j];
          base += c + j * groups < chunk ? v[j] : 0;
        }
      }
      for (; c < num_chunks; c += groups) {
        const int v = a.chunk_counts[static_cast<int64_t>(c) * E + e];
        tot += v;
        base += c < chunk ? v : 0;
      }
      s_ptot[g * E + e] = tot;
      s_pbase[g * E + e] = base;
    }
    __syncthreads();
    for (int e = tid; e < E; e += kChunkThreads) {
      int tot = 0, base = 0;
      for (int g = 0; g < groups; ++g) {
        tot += s_ptot[g * E + e];
        base += s_pbase[g * E + e];
      }
      s_tot[e] = tot;
      s_cbase[e] = base;
    }
    __syncthreads();
  }
  publish_offsets(a, s_tot, s_off, chunk == 0);
  const int64_t ntasks =
      static_cast<int64_t>(effective_tokens(a.runtime_tokens, a.host_tokens)) * a.topk;
  const WaveRange wr = chunk_wave_range(ntasks, chunk, chunk_tasks, wave);
  // the count kernel's per-wave counts of this chunk (same task split), else count again
  const bool counted = a.wave_counts != nullptr;
  const int32_t* wsrc = counted ? a.wave_counts + static_cast<int64_t>(chunk) * kChunkWaves * E : nullptr;
  for (int i = tid; i < kChunkWaves * E; i += kChunkThreads) s_wbase[i / E][i % E] = counted ? wsrc[i] : 0;
  __syncthreads();
  wave_route(a, wr.begin, wr.end, s_wbase[wave], [&]() {
    __syncthreads();
    for (int e = tid; e < E; e += kChunkThreads) {
      int run = s_off[e] + s_cbase[e];
      for (int w = 0; w < kChunkWaves; ++w) {
        const int c = s_wbase[w][e];
        s_wbase[w][e] = run;
        run += c;
      }
    }
    __syncthreads();
  }, counted);
}

}  // namespace

int64_t route_chunk_tasks(int64_t ntasks) {
  // <= 256 chunks (one workgroup each), at least 1024 tasks per chunk, multiple of 1024
  int64_t chunk = (ntasks + 255) / 256;
  chunk = (chunk + kRouteChunk - 1) / kRouteChunk * kRouteChunk;
  return chunk < kRouteChunk ? kRouteChunk : chunk;
}

hipError_t launch_route(const RouteArgs& a, int64_t max_tasks, hipStream_t stream) {
  if (max_tasks <= 0) return hipSuccess;
  if (max_tasks <= kSmallWaves * kRouteChunk && a.num_experts <= kSmallMaxExperts) {
    return launch_kernel(route_small_kernel, dim3(1), dim3(kSmallThreads), 0, stream, a);
  }
  const int64_t chunk = route_chunk_tasks(max_tasks);
  const int64_t chunks = (max_tasks + chunk - 1) / chunk;
  const hipError_t err = launch_kernel(route_count_kernel, dim3(static_cast<unsigned>(chunks)),
                                       dim3(kChunkThreads), 0, stream, a, static_cast<int>(chunk));
  if (err != hipSuccess) return err;
  return launch_kernel(route_chunk_scatter_kernel, dim3(static_cast<unsigned>(chunks)),
                       dim3(kChunkThreads), 0, stream, a, static_cast<int>(chunk),
                       static_cast<int>(chunks));
}

}  // namespace mmoe
