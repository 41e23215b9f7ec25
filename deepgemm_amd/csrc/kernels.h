// kernels.h -- host-side launch interfaces of the gfx950 kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmoe {

constexpr int kRouteChunk = 1024;  // tasks per routing chunk (== MMOE_ROUTE_CHUNK)
constexpr int kRouteWaves = 16;    // waves of a routing chunk's workgroup
constexpr int kMaxExperts = 1024;  // LDS-resident per-expert tables in the routing kernels

struct RouteArgs {
  const void* topk_idx;           // int64 or int32 [S, K]
  int idx_i64;
  const float* topk_w;            // f32 [S, K]
  const int32_t* runtime_tokens;  // device scalar or null
  int host_tokens;                // S (upper bound when runtime_tokens is set)
  int topk;
  int num_experts;
  int check_weight;               // forward rule: w != 0 required
  int64_t row_cap;                // rows >= row_cap are dropped (output_index = -1)
  int32_t* chunk_counts;          // [nchunks, E] per-chunk counts (large launches only)
  int32_t* wave_counts;           // [nchunks, kRouteWaves, E] per-wave counts of each chunk
                                  // (large launches), or null: the scatter counts again
  int32_t* counts;                // [E]
  int32_t* offsets;               // [E+1]
  int32_t* meta;                  // [16]; meta[0] = R
  int32_t* stats;                 // [E] or null (+= counts)
  const int32_t* given_counts;    // preprocess: offsets from caller counts, else null
  int32_t* output_index;          // [S, K]
  int32_t* row_token;             // [rows]
  float* row_weight;              // [rows] or null
  int32_t* m_indices;             // [rows] or null
  int32_t* zero_ints;             // zeroed by the routing launch (the GEMMs' claim counters), or null
  int zero_count;
  int64_t fused_max_tasks;        // > 0: the launch returns at once when the live tasks are at
                                  // most this many (GEMM1 then routes them in-kernel)
};

// Count -> offsets -> stable scatter over at most max_tasks = S*K tasks. Deterministic: rows
// of an expert in ascending task order. chunk_counts needs ceil(max_tasks/kRouteChunk)*E ints,
// wave_counts kRouteWaves times as many (route_count_ints gives both together).
hipError_t launch_route(const RouteArgs& a, int64_t max_tasks, hipStream_t stream);
inline int64_t route_count_ints(int64_t max_tasks, int num_experts) {
  const int64_t chunks = (max_tasks + kRouteChunk - 1) / kRouteChunk;
  return (chunks > 0 ? chunks : 1) * num_experts * (1 + kRouteWaves);
}

// Per-expert tile engine of the grouped GEMM: kAuto picks STREAM for experts with <= 128 rows
// (weight streaming, decode) and TILE otherwise (256x256 MFMA tiles, prefill).
enum class GemmEngine : int { kAuto = 0, kStream = 1, kTile = 2 };

// Fused GEMM1 epilogue: SwiGLU x route weight -> bf16 y.
struct SwigluEpilogue {
  int enabled;
  int inter;                // I: gate weight rows [0, I), up rows [I, 2I)
  const float* row_weight;  // [rows] top-k weight of each routed row
  uint16_t* y;              // bf16 [rows, I] SwiGLU x weight output (before the requant)
  int has_clamp;
  float clamp;
};

// WIDE GEMMs (ZeroFill::y set): the y rows of tokens without a valid routed slot are zeros, and
// a workgroup that has run out of tiles writes them while others still run tiles (the kernel's
// end leaves workgroups idle), kZeroFillTokens tokens at a time claimed from *claim (GEMM1
// first, GEMM2 goes on from where it stopped); *idle counts the kernel's workgroups out of
// tiles. The routing launch of the same call zeroes the counters. The combine then skips those
// tokens in the chunks claimed (CombineArgs::zfill_claim). y null: off.
constexpr int kZeroFillTokens = 64;
struct ZeroFill {
  uint16_t* y;                  // bf16 [S, hidden]
  int32_t* claim;
  int32_t* idle;
  const int32_t* output_index;  // [S, topk]
  const int32_t* runtime_tokens;
  int host_tokens, topk, hidden;
};

struct GemmArgs {
  const uint8_t* a;          // e4m3 rows, row-major, lda bytes apart
  const int32_t* row_token;  // non-null: A row r is a[row_token[r]] (gather), scale a_scale[token]
  const float* a_scale;      // per token (gather) or per row
  int64_t lda;
  const uint8_t* b;          // e4m3 Marlin [E, N/16, K*16]
  const float* b_scale;      // f32 [E, N]
  uint16_t* c;               // bf16 [rows, N]
  const int32_t* counts;     // [E]
  const int32_t* offsets;    // [E+1]
  int num_experts;
  int n;
  int k;
  GemmEngine engine;
  SwigluEpilogue sw;         // GEMM1 only (requires row_token); c is unused then
  int route_in_kernel;       // GEMM1: 1 = route the tasks in the kernel (<= gemm_route_max_tasks()),
                             // 2 = only when the live tasks are at most that many
  RouteArgs route;           // the routing to do then (counts, offsets, row tables are written)
  // GEMM2 on the WIDE kernel, when *direct_flag != 0: rows with row_dest[r] >= 0 go to
  // y_direct[row_dest[r]] (bf16 [S, N], a negative zero stored as +0 like the combine's sum)
  // instead of c. Null pointers: every row to c.
  const int32_t* row_dest;
  uint16_t* y_direct;
  const int32_t* direct_flag;
  // WIDE kernel work claiming (kSchedInts ints, zero at launch; the kernel leaves them zero):
  // [0..7] per-XCD claim counters, [8] finished workgroups. Null: static dealing.
  int32_t* sched;
  ZeroFill zf;  // WIDE kernels only
  // Set by launch_grouped_gemm for a row bound that selects the WIDE kernel while the actual rows
  // are only known on the device (graph replays): the 8-wave and the WIDE kernel are both
  // launched, and each returns at once unless the routed rows (*dual_rows, the routing's
  // meta[0], or its meta[4] for eager calls) select it -- WIDE at dual_min_rows or more.
  // Null: the launch always runs.
  const int32_t* dual_rows;
  int dual_min_rows;
  // Decode pipeline GEMM1: per row, the max |SwiGLU output| of each 64-column unit (float
  // [rows, n / 64]), which the pipeline's requant takes its row maxima from. Null: not written.
  float* row_pmax;
};
constexpr int kSchedInts = 16;
constexpr int kZeroFillClaim = 9;  // GEMM1's sched int 9: ZeroFill::claim; 10, 11: the GEMMs' idle

// Grouped FP8 GEMM over expert-contiguous rows: c[r, n] = bf16((sum_k a[r,k] b[e,n,k]) *
// a_scale[r] * b_scale[e,n]). Persistent: the grid strides over the tiles, enumerated on the
// device from counts (max_rows bounds the grid only). With rows_on_device (the routing's
// meta[0]) and a bound that selects the WIDE kernel, the kernel is chosen on the device from
// the routed rows instead (GemmArgs::dual_rows).
// With route_small_in_kernel (a GEMM1 on device-read tokens whose bound is too large for
// in-kernel routing), the 8-wave kernel routes the tasks itself when the live ones fit
// (route_in_kernel 2); the call's routing launch then returns at once
// (RouteArgs::fused_max_tasks).
hipError_t launch_grouped_gemm(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream,
                               const int32_t* rows_on_device = nullptr,
                               bool route_small_in_kernel = false, int dual_min_rows = 0);
// The routed-row count from which the WIDE kernel is chosen on the device (dual launches of
// graph replays; dual_min_rows 0 selects it).
int gemm_wide_min_rows(int num_experts);
// Eager calls on the auto schedule: true when the row bound selects WIDE but the routed rows
// should choose on the device (a dual launch with rows_on_device = the routing's meta[4], the
// largest expert's row count, and dual_min_rows = gemm_eager_dual_min_largest: WIDE once an
// expert has more than 128 rows).
bool gemm_eager_dual(const GemmArgs& g, int max_rows);
int gemm_eager_dual_min_largest();
bool gemm_shape_supported(int n, int k);
// True when launch_grouped_gemm runs the WIDE kernel for g (the choice depends only on the
// shape and the row bound, so separate stage calls agree on it).
bool gemm_wide_selected(const GemmArgs& g, int max_rows);
// Largest task count (S*K) and expert count GEMM1 can route in-kernel.
int gemm_route_max_tasks();
int gemm_route_max_experts();

// Rows whose token has exactly one routed slot: their GEMM2 output is the layer output (the
// combine's one-term sum), so GEMM2 can write it straight into y. row_dest[r] = the token of
// row r if so, else -1 (built by the requant from output_index); *meta_flag = 1 when built,
// 0 when not (GEMM2 and the combine read it).
struct RowDest {
  int32_t* row_dest;             // [rows] or null (not built)
  const int32_t* row_token;      // [rows]
  const int32_t* output_index;   // [S, K]
  int topk;
  int32_t* meta_flag;
};

// Per-row requant of the SwiGLU output: amax = max |y| (written out), a = max(amax, 1e-4);
// act = e4m3(clip(y * 448/a)); act_scale = a/448 -- for rows < meta[0]. y is GEMM1's SwiGLU x
// route weight output, bf16 [rows, I]. meta[1] records whether the WIDE GEMM1 ran (wide). With
// dest.row_dest it also builds the direct-write table (RowDest). With dual_rows (a dual GEMM1
// launch): wide is decided on the device, true when *dual_rows >= dual_min_rows, and the
// direct-write table is built only then.
hipError_t launch_requant(const uint16_t* src, bool wide, float* amax, int32_t* meta, uint8_t* act,
                          float* act_scale, int64_t max_rows, int inter, const RowDest& dest,
                          int num_cus, hipStream_t stream, const int32_t* dual_rows = nullptr,
                          int dual_min_rows = 0);

struct CombineArgs {
  uint16_t* y;                     // bf16 [S, H]
  const uint16_t* part;            // bf16 [rows, H]
  const int32_t* skip_single;      // null, or *skip_single != 0: tokens with exactly one
                                   // routed slot were written by GEMM2 (RowDest)
  const int32_t* output_index;     // [S, K]
  const void* topk_ids;            // optional validity/weight source (postprocess)
  int ids_i64;
  const float* topk_w;             // applied when apply_weights
  int apply_weights;
  const int32_t* runtime_tokens;
  int host_tokens;
  int topk;
  int hidden;
  // the ZeroFill claim counter of this call's WIDE GEMM1: tokens without a routed slot in the
  // chunks it counts have their zero rows already. Null: the combine writes every zero row.
  const int32_t* zfill_claim;
};
hipError_t launch_combine(const CombineArgs& c, int num_cus, hipStream_t stream);

// Decode pipeline (gemm.hip): GEMM1 with the in-kernel routing, the requant, GEMM2 of the
// streaming engine and (PipeArgs::y) the combine in one launch, each group of rows handed from
// GEMM1 to GEMM2 inside its XCD, each token combined once its experts' GEMM2 items are done.
// pipe: kPipeInts counters, zero when the launch starts (its last workgroup to leave zeroes
// them again), each header counter in a 128-byte line of its own (every workgroup goes to them
// at about the same time): the per-XCD claim counters at x * kPipeLine, the count of workgroups
// that ran out of items at kPipeFinishAt, the count of workgroups that left at kPipeExitAt
// (the count of bounded waits that ran out next to it, at kPipeFailAt: rarely touched; the last
// workgroup to leave copies it to meta[3]); then GEMM1 items done per group ([kPipeDone1At..],
// kMaxPipeGroups) and GEMM2 items done per expert (expert e's at kPipeDone2At + e *
// kPipeDone2Stride: the combine's waves poll them).
constexpr int kPipeXcds = 8;
constexpr int kPipeLine = 32;
constexpr int kPipeFinishAt = kPipeXcds * kPipeLine;
constexpr int kPipeExitAt = (kPipeXcds + 1) * kPipeLine;
constexpr int kPipeFailAt = kPipeExitAt + 1;
// Polls of a bounded wait (a group's or an expert's count; far longer than any item). A wait
// that runs out counts itself and goes on, so the launch always ends; the call's status
// (meta[3], mmoe_scratch_status) then reports that its output is not valid.
constexpr int kPipeSpinLimit = 1 << 20;
constexpr int kPipeHeader = (kPipeXcds + 2) * kPipeLine;
constexpr int kMaxPipeGroups = 512;  // groups of <= 64 rows: S*K <= 8192 rows over <= 255 experts
constexpr int kMaxPipeExperts = 256;
constexpr int kPipeDone1At = kPipeHeader;
constexpr int kPipeDone2At = kPipeHeader + kMaxPipeGroups;
constexpr int kPipeDone2Stride = 16;
constexpr int kPipeInts = kPipeHeader + kMaxPipeGroups + kMaxPipeExperts * kPipeDone2Stride;
struct PipeArgs {
  GemmArgs g1;           // GEMM1: route_in_kernel 1, SwiGLU epilogue into the bf16 y
  GemmArgs g2;           // GEMM2: a = act, a_scale = act_scale, c = the bf16 partial rows
  uint8_t* act;          // e4m3 [rows, I] (written by the first GEMM2 item of each group)
  float* act_scale;      // [rows]
  float* amax;           // [rows] (with act)
  int32_t* meta;         // [1] = 0 (the requant read y); [3] = bounded waits that ran out
                         // (written at the end of the launch)
  int32_t* direct_flag;  // set to 0 (no direct rows), or null
  int32_t* pipe;
  uint16_t* y;           // non-null: the launch also runs the combine into y (bf16 [S, H];
                         // H % 8 == 0 and H <= kPipeCombineMaxHidden)
  int spin_limit;        // polls of a bounded wait: kPipeSpinLimit, or 0 to test the error path
                         // (every wait then gives up at once)
};
constexpr int kPipeCombineMaxHidden = 64 * 8 * 8;  // one wave a token: 8 16-byte groups a lane
bool decode_pipeline_supported(const GemmArgs& g1, const GemmArgs& g2, int num_cus);
hipError_t launch_decode_pipeline(const PipeArgs& p, int num_cus, hipStream_t stream);

// For every task (token t, slot s) with row = output_index[t*K+s] >= 0:
// grouped_x[row] = x[t], grouped_scale[row] = x_sf[t].
hipError_t launch_gather_tasks(uint8_t* grouped_x, float* grouped_scale, const uint8_t* x,
                               const float* x_sf, const int32_t* output_index, int64_t tasks,
                               int topk, int hidden, hipStream_t stream);

hipError_t launch_cast_fp8_channelwise(uint8_t* out, float* scale, const uint16_t* x,
                                       int64_t rows, int64_t cols, hipStream_t stream);
hipError_t launch_marlin_pack(uint8_t* out, const uint8_t* in, int64_t groups, int64_t rows,
                              int64_t k, hipStream_t stream);
hipError_t launch_f32_to_e4m3(uint8_t* out, const float* in, int64_t n, hipStream_t stream);

}  // namespace mmoe
