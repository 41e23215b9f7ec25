// route_wave.cuh -- wave-level building blocks of the deterministic routing, shared by the
// routing kernels (route.hip) and the grouped GEMM's in-kernel routing (gemm.hip).
//
// A task (token t, slot s) goes to local expert e = topk_idx[t,s] iff 0 <= e < E and, for the
// layer, topk_weights[t,s] != 0 (deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:352).
// Within an expert, rows follow ascending task index. Ranks come from wave ballots: one ballot
// per bit of the expert id gives every lane the mask of lanes holding the same expert (a
// match-any in log2(E) votes); a lane's rank is the popcount of that mask below it.
#pragma once

#include "common.cuh"
#include "kernels.h"

namespace mmoe {

// Expert of a task (or -1), from already-loaded id and weight.
__device__ __forceinline__ int valid_expert(const RouteArgs& a, int64_t e, float w) {
  if (e < 0 || e >= a.num_experts) return -1;
  if (a.check_weight && w == 0.0f) return -1;
  return static_cast<int>(e);
}

__device__ __forceinline__ uint64_t lanes_below() {
  const int lane = lane_id();
  return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

__device__ __forceinline__ int expert_id_bits(int num_experts) {
  int bits = 0;
  while ((1 << bits) < num_experts) ++bits;
  return bits;
}

// Loads P passes of 64 tasks starting at `begin` (task begin + p*64 + lane) into registers,
// all loads issued before any is used (one memory round trip per batch). The id width is a
// branch around the whole batch: a width test per load placed a wait inside every branch, and
// the batch's loads went out one round trip at a time.
template <int P, typename Id>
__device__ __forceinline__ void wave_load_ids(const Id* idx, const float* topk_w, int64_t begin,
                                              int64_t end, int64_t* ids, float* wv) {
  const int lane = lane_id();
  Id raw[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int64_t task = begin + p * kWave + lane;
    const int64_t t = task < end ? task : 0;
    raw[p] = idx[t];
    wv[p] = topk_w[t];
  }
#pragma unroll
  for (int p = 0; p < P; ++p) ids[p] = begin + p * kWave + lane < end ? static_cast<int64_t>(raw[p]) : -1;
}

template <int P>
__device__ __forceinline__ void wave_load(const RouteArgs& a, int64_t begin, int64_t end, int* ev,
                                          float* wv) {
  int64_t ids[P];
  if (a.idx_i64)
    wave_load_ids<P>(static_cast<const int64_t*>(a.topk_idx), a.topk_w, begin, end, ids, wv);
  else
    wave_load_ids<P>(static_cast<const int32_t*>(a.topk_idx), a.topk_w, begin, end, ids, wv);
#pragma unroll
  for (int p = 0; p < P; ++p) ev[p] = valid_expert(a, ids[p], wv[p]);
}

// Lanes of the wave holding the same expert id as this lane (invalid lanes: none), from one
// ballot per id bit: O(log2 E) wave votes, no loop over the distinct experts.
__device__ __forceinline__ uint64_t match_expert(int e, int id_bits) {
  const uint64_t valid = __ballot(e >= 0);
  uint64_t m = valid;
  for (int b = 0; b < id_bits; ++b) {
    const uint64_t ones = __ballot(e >= 0 && ((e >> b) & 1));
    m &= ((e >> b) & 1) ? ones : ~ones;
  }
  return e >= 0 ? m : 0ull;
}

// Adds the per-expert counts of one 64-task pass into cnt[e] (this wave's private row): the
// lowest lane of every equal-expert group adds the group size.
__device__ __forceinline__ void wave_count_pass(int e, int id_bits, int* cnt) {
  const uint64_t m = match_expert(e, id_bits);
  if (e >= 0 && (m & lanes_below()) == 0ull) cnt[e] += __popcll(m);
  __builtin_amdgcn_wave_barrier();
}

}  // namespace mmoe
