// capi.hip -- the C ABI (include/megamoe_hip.h): validation, workspace layout, schedule choice
// and the stream-ordered launch sequence of the layer. No allocation, no host synchronisation.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "../../include/megamoe_hip.h"
#include "kernels.h"
#include "launch.h"

namespace {

constexpr int kTokenAlignment = 384;  // deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:9
constexpr int kMaxTopk = 16;
constexpr int kMaxLayerExperts = 256;  // per-expert tile tables of the grouped GEMM
// The kernels count routed rows (tokens x top-k) in 32-bit integers.
constexpr int64_t kMaxRoutedRows = int64_t{1} << 30;

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

int check_common(int num_ranks, int num_experts, int num_max_tokens, int num_topk, int hidden,
                 int intermediate) {
  if (num_ranks <= 0) return MMOE_ERR_NUM_RANKS;
  if (num_experts % num_ranks != 0) return MMOE_ERR_EXPERTS_DIVISIBLE;
  if (hidden <= 0 || intermediate <= 0) return MMOE_ERR_HIDDEN_SIZES;
  if (num_max_tokens < 0) return MMOE_ERR_ARGUMENT;
  if (num_topk <= 0 || num_topk > kMaxTopk) return MMOE_ERR_TOPK;
  if (num_experts / num_ranks <= 0 || num_experts / num_ranks > mmoe::kMaxExperts)
    return MMOE_ERR_UNSUPPORTED_SHAPE;
  if (static_cast<int64_t>(num_max_tokens) * num_topk > kMaxRoutedRows) return MMOE_ERR_UNSUPPORTED_SHAPE;
  return MMOE_OK;
}

void plan_scratch(int num_ranks, int num_experts, int num_max_tokens, int num_topk, int hidden,
                  int intermediate, mmoe_scratch_layout* l) {
  const int64_t e_local = num_experts / num_ranks;
  const int64_t tasks = static_cast<int64_t>(num_max_tokens) * num_topk;
  const int64_t rows = align_up(tasks > 0 ? tasks : 1, 256);
  const int64_t chunks = (tasks + mmoe::kRouteChunk - 1) / mmoe::kRouteChunk;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  memset(l, 0, sizeof(*l));
  l->row_capacity = rows;
  l->num_chunks = chunks;
  // The decode pipeline's counters and meta come first, at offsets that no shape changes: the
  // counters must read zero when a call starts and every call leaves them zero, so a scratch
  // reused across shapes (or the static one) never hands a call another section's bytes as
  // counters; meta[3] (the status) sits where mmoe_scratch_status finds it without the shape.
  l->pipe_offset = take(mmoe::kPipeInts * 4);
  l->meta_offset = take(16 * 4);
  l->counts_offset = take(e_local * 4);
  l->offsets_offset = take((e_local + 1) * 4);
  l->chunk_counts_offset = take(mmoe::route_count_ints(tasks, static_cast<int>(e_local)) * 4);
  l->output_index_offset = take((tasks > 0 ? tasks : 1) * 4);
  l->row_token_offset = take(rows * 4);
  l->row_weight_offset = take(rows * 4);
  l->m_indices_offset = take(rows * 4);
  l->act_scale_offset = take(rows * 4);
  l->amax_offset = take(rows * 4);
  l->y_offset = take(rows * static_cast<int64_t>(intermediate) * 2);
  l->act_offset = take(rows * static_cast<int64_t>(intermediate));
  l->part_offset = take(rows * static_cast<int64_t>(hidden) * 2);
  l->row_dest_offset = take(rows * 4);
  l->sched_offset = take(2 * mmoe::kSchedInts * 4);
  l->pmax_offset = take(std::min<int64_t>(rows, mmoe::gemm_route_max_tasks()) *
                        (2 * static_cast<int64_t>(intermediate) / 64) * 4);
  l->total_bytes = off;
}

void plan_symm(int num_max_tokens, int num_topk, int hidden, mmoe_symm_layout* s) {
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  memset(s, 0, sizeof(*s));
  const int64_t t = num_max_tokens;
  s->runtime_num_tokens_offset = take(16);
  s->x_offset = take(t * hidden);
  s->x_sf_offset = take(t * 4);
  s->topk_idx_offset = take(t * num_topk * 8);
  s->topk_weights_offset = take(t * num_topk * 4);
  s->total_bytes = off;
}

std::atomic<int> g_cu_cache[64];

int device_cus(int* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MMOE_ERR_NO_DEVICE;
  if (dev >= 0 && dev < 64) {
    const int cached = g_cu_cache[dev].load(std::memory_order_relaxed);
    if (cached > 0) {
      *out = cached;
      return MMOE_OK;
    }
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return MMOE_ERR_NO_DEVICE;
  if (dev >= 0 && dev < 64) g_cu_cache[dev].store(cus, std::memory_order_relaxed);
  *out = cus;
  return MMOE_OK;
}

template <class T>
T* at(void* base, int64_t off) {
  return reinterpret_cast<T*>(static_cast<uint8_t*>(base) + off);
}

int validate_forward(const mmoe_forward_args* a) {
  if (a == nullptr) return MMOE_ERR_NULL_POINTER;
  int st = check_common(1, a->num_experts, a->num_max_tokens, a->num_topk, a->hidden,
                        a->intermediate);
  if (st != MMOE_OK) return st;
  if (a->hidden % 16 || a->intermediate % 16) return MMOE_ERR_MARLIN_DIVISIBLE;
  if (a->num_experts > kMaxLayerExperts) return MMOE_ERR_UNSUPPORTED_SHAPE;
  if (a->num_tokens < 0) return MMOE_ERR_ARGUMENT;
  if (a->num_tokens > a->num_max_tokens) return MMOE_ERR_TOO_MANY_TOKENS;
  if (!mmoe::gemm_shape_supported(2 * a->intermediate, a->hidden) ||
      !mmoe::gemm_shape_supported(a->hidden, a->intermediate))
    return MMOE_ERR_UNSUPPORTED_SHAPE;
  if (a->schedule < MMOE_SCHEDULE_AUTO || a->schedule > MMOE_SCHEDULE_STAGED)
    return MMOE_ERR_SCHEDULE;
  if ((a->debug_flags & ~MMOE_DEBUG_NO_WAIT) != 0) return MMOE_ERR_ARGUMENT;
  mmoe_symm_layout sl;
  plan_symm(a->num_max_tokens, a->num_topk, a->hidden, &sl);
  if (a->sym_buffer_bytes >= 0 && a->sym_buffer_bytes < sl.total_bytes)
    return MMOE_ERR_SYM_BUFFER_SMALL;
  mmoe_scratch_layout l;
  plan_scratch(1, a->num_experts, a->num_max_tokens, a->num_topk, a->hidden, a->intermediate,
               &l);
  if (a->route_scratch_bytes < l.total_bytes) return MMOE_ERR_SCRATCH_SMALL;
  if (a->num_tokens > 0 &&
      (a->y == nullptr || a->x == nullptr || a->x_sf == nullptr || a->topk_idx == nullptr ||
       a->topk_weights == nullptr || a->w1 == nullptr || a->w1_sf == nullptr ||
       a->w2 == nullptr || a->w2_sf == nullptr || a->route_scratch == nullptr))
    return MMOE_ERR_NULL_POINTER;
  return MMOE_OK;
}

mmoe::RouteArgs forward_route_args(const mmoe_forward_args* a, const mmoe_scratch_layout& l) {
  mmoe::RouteArgs r;
  memset(&r, 0, sizeof(r));
  void* ws = a->route_scratch;
  r.topk_idx = a->topk_idx;
  r.idx_i64 = 1;
  r.topk_w = a->topk_weights;
  r.runtime_tokens = a->runtime_num_tokens;
  r.host_tokens = a->num_tokens;
  r.topk = a->num_topk;
  r.num_experts = a->num_experts;
  r.check_weight = 1;
  r.row_cap = l.row_capacity;
  r.chunk_counts = at<int32_t>(ws, l.chunk_counts_offset);
  r.wave_counts = r.chunk_counts + (l.num_chunks > 0 ? l.num_chunks : 1) * a->num_experts;
  r.counts = at<int32_t>(ws, l.counts_offset);
  r.offsets = at<int32_t>(ws, l.offsets_offset);
  r.meta = at<int32_t>(ws, l.meta_offset);
  r.stats = a->stats;
  r.given_counts = nullptr;
  r.output_index = at<int32_t>(ws, l.output_index_offset);
  r.row_token = at<int32_t>(ws, l.row_token_offset);
  r.row_weight = at<float>(ws, l.row_weight_offset);
  r.m_indices = at<int32_t>(ws, l.m_indices_offset);
  r.zero_ints = at<int32_t>(ws, l.sched_offset);  // the GEMMs' claim counters start at zero
  r.zero_count = 2 * mmoe::kSchedInts;
  return r;
}

// ---- scratch of the allocation-free entry point (mmoe_forward_static) ----
// A file-scope device array: each GPU the library runs on holds its own copy, at its own
// address, from the code object's load until the process ends. In host code `scratch` is a
// host-side stand-in, never a device address: the device address comes from
// hipGetSymbolAddress, once per device, and only that pointer reaches kernels.
static __device__ __align__(256) uint8_t scratch[MMOE_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_static_scratch[kMaxDevices];
std::mutex g_static_scratch_mu;

// The current device's address of `scratch` (set up on the first call on that device).
int static_scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MMOE_ERR_NO_DEVICE;
  void* p = g_static_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_static_scratch_mu);
    p = g_static_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
        return MMOE_ERR_HIP;
      g_static_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MMOE_OK;
}

// mmoe_forward_profile: the stage that the following launches of this host thread belong to.
void mark_stage(int stage) {
  if (mmoe::LaunchTimer* t = mmoe::launch_timer()) t->stage = stage;
}

int run_route(const mmoe_forward_args* a, const mmoe_scratch_layout& l, hipStream_t s) {
  const mmoe::RouteArgs r = forward_route_args(a, l);
  const int64_t tasks = static_cast<int64_t>(a->num_tokens) * a->num_topk;
  return mmoe::launch_route(r, tasks, s) == hipSuccess ? MMOE_OK : MMOE_ERR_HIP;
}

}  // namespace

namespace mmoe {
LaunchTimer*& launch_timer() {
  static thread_local LaunchTimer* timer = nullptr;
  return timer;
}
}  // namespace mmoe

extern "C" {

int mmoe_token_alignment(void) { return kTokenAlignment; }

int mmoe_symm_buffer_layout(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                            int hidden, int intermediate, mmoe_symm_layout* out) {
  if (out == nullptr) return MMOE_ERR_NULL_POINTER;
  const int st = check_common(num_ranks, num_experts, num_max_tokens, num_topk, hidden,
                              intermediate);
  if (st != MMOE_OK) return st;
  plan_symm(num_max_tokens, num_topk, hidden, out);
  return MMOE_OK;
}

int mmoe_route_scratch_layout(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                              int hidden, int intermediate, mmoe_scratch_layout* out) {
  if (out == nullptr) return MMOE_ERR_NULL_POINTER;
  const int st = check_common(num_ranks, num_experts, num_max_tokens, num_topk, hidden,
                              intermediate);
  if (st != MMOE_OK) return st;
  plan_scratch(num_ranks, num_experts, num_max_tokens, num_topk, hidden, intermediate, out);
  return MMOE_OK;
}

int mmoe_route_scratch_bytes(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                             int hidden, int intermediate, int64_t* out_bytes) {
  if (out_bytes == nullptr) return MMOE_ERR_NULL_POINTER;
  mmoe_scratch_layout l;
  const int st = mmoe_route_scratch_layout(num_ranks, num_experts, num_max_tokens, num_topk,
                                           hidden, intermediate, &l);
  if (st != MMOE_OK) return st;
  *out_bytes = l.total_bytes;
  return MMOE_OK;
}

const char* mmoe_build_config(void) {
  return "{\"operator\": \"fp8_w8a8_mega_moe\", \"package\": \"megamoe\", "
         "\"arch\": \"gfx950\", \"fp8_format\": \"e4m3fn (OCP)\", "
         "\"weight_scale_mode\": \"channelwise_fp32\", \"input_scale_mode\": "
         "\"channelwise_fp32\", \"l2_act_scale_mode\": \"channelwise_fp32\", "
         "\"has_fp8_api\": true, \"has_fp4_api\": false, \"mfma\": "
         "\"v_mfma_f32_32x32x64_f8f6f4\", \"fusion_boundary\": "
         "\"route|gemm1(gather)|swiglu_quant|gemm2|combine\", \"num_ranks\": 1}";
}

const char* mmoe_status_string(int status) {
  switch (status) {
    case MMOE_OK: return "ok";
    case MMOE_ERR_NULL_POINTER: return "a required pointer is null";
    case MMOE_ERR_NUM_RANKS: return "num_ranks must be positive";
    case MMOE_ERR_EXPERTS_DIVISIBLE: return "num_experts must be divisible by num_ranks";
    case MMOE_ERR_HIDDEN_SIZES: return "hidden sizes must be positive";
    case MMOE_ERR_MARLIN_DIVISIBLE:
      return "DCU MegaMoE Marlin weights require rows and K divisible by 16";
    case MMOE_ERR_TOO_MANY_TOKENS: return "too many tokens";
    case MMOE_ERR_SYM_BUFFER_SMALL:
      return "sym_buffer is too small for the requested DCU MegaMoE capacity";
    case MMOE_ERR_SCRATCH_SMALL:
      return "route_scratch is too small for the requested DCU MegaMoE capacity";
    case MMOE_ERR_UNSUPPORTED_SHAPE:
      return "unsupported shape: hidden and intermediate must be multiples of 128, "
             "1 <= local experts <= 1024 (256 for a forward call), num_max_tokens * num_topk <= 2^30";
    case MMOE_ERR_TOPK: return "num_topk must be in 1..16";
    case MMOE_ERR_SCHEDULE: return "unknown schedule override";
    case MMOE_ERR_HIP: return "HIP kernel launch failed";
    case MMOE_ERR_NO_DEVICE: return "no usable HIP device";
    case MMOE_ERR_ARGUMENT: return "invalid argument";
    case MMOE_ERR_STATIC_SCRATCH:
      return "mmoe_forward_static: the call needs more scratch than the static buffer's "
             "MMOE_STATIC_SCRATCH_BYTES (128 MiB); call mmoe_forward with a route_scratch";
    default: return "unknown status";
  }
}

int mmoe_route(const mmoe_forward_args* a, void* stream) {
  const int st = validate_forward(a);
  if (st != MMOE_OK) return st;
  mmoe_scratch_layout l;
  plan_scratch(1, a->num_experts, a->num_max_tokens, a->num_topk, a->hidden, a->intermediate,
               &l);
  if (a->num_tokens == 0) return MMOE_OK;
  return run_route(a, l, static_cast<hipStream_t>(stream));
}

int mmoe_forward_stages(const mmoe_forward_args* a, int first_stage, int last_stage,
                        void* stream) {
  int st = validate_forward(a);
  if (st != MMOE_OK) return st;
  if (first_stage < MMOE_STAGE_ROUTE || last_stage > MMOE_STAGE_COMBINE ||
      first_stage > last_stage)
    return MMOE_ERR_ARGUMENT;
  if (a->num_tokens == 0) return MMOE_OK;
  int cus = 0;
  st = device_cus(&cus);
  if (st != MMOE_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  mmoe_scratch_layout l;
  plan_scratch(1, a->num_experts, a->num_max_tokens, a->num_topk, a->hidden, a->intermediate,
               &l);
  auto runs = [&](int stage) { return first_stage <= stage && stage <= last_stage; };

  // AUTO: the engine is chosen per expert on the device from its routed rows (the row count is
  // only known there); PERSISTENT / STAGED force the streaming / tiled engine for every expert.
  const mmoe::GemmEngine engine = a->schedule == MMOE_SCHEDULE_PERSISTENT ? mmoe::GemmEngine::kStream
                                  : a->schedule == MMOE_SCHEDULE_STAGED   ? mmoe::GemmEngine::kTile
                                                                          : mmoe::GemmEngine::kAuto;
  const int max_rows = a->num_tokens * a->num_topk;
  void* ws = a->route_scratch;

  // Small task counts: GEMM1 routes in-kernel (one launch fewer, no single-workgroup routing
  // latency); the routing kernels serve larger counts and a routing-only call.
  const bool route_in_gemm1 = runs(MMOE_STAGE_ROUTE) && runs(MMOE_STAGE_GEMM1) &&
                              max_rows <= mmoe::gemm_route_max_tasks() &&
                              a->num_experts <= mmoe::gemm_route_max_experts();
  // Graph replays (tokens read on the device) with a bound that selects the WIDE kernels: the
  // routed rows choose between those and the 8-wave kernels on the device, so a replay with
  // few live tokens in a large bucket still runs the decode engines; and when GEMM1 and the
  // routing run together, the 8-wave GEMM1 also routes the live tasks itself when they fit
  // (the routing launch then returns at once).
  const int32_t* rows_on_device =
      a->runtime_num_tokens != nullptr ? at<int32_t>(ws, l.meta_offset) : nullptr;
  const bool route_small_in_gemm1 = rows_on_device != nullptr && !route_in_gemm1 &&
                                    runs(MMOE_STAGE_ROUTE) && runs(MMOE_STAGE_GEMM1) &&
                                    a->num_experts <= mmoe::gemm_route_max_experts();
  if (runs(MMOE_STAGE_ROUTE) && !route_in_gemm1) {
    mark_stage(MMOE_STAGE_ROUTE);
    mmoe::RouteArgs r = forward_route_args(a, l);
    const int64_t tasks = static_cast<int64_t>(a->num_tokens) * a->num_topk;
    if (route_small_in_gemm1) r.fused_max_tasks = mmoe::gemm_route_max_tasks();
    if (mmoe::launch_route(r, tasks, s) != hipSuccess) return MMOE_ERR_HIP;
  }

  mmoe::GemmArgs g1;
  memset(&g1, 0, sizeof(g1));
  g1.a = static_cast<const uint8_t*>(a->x);
  g1.row_token = at<int32_t>(ws, l.row_token_offset);
  g1.a_scale = a->x_sf;
  g1.lda = a->hidden;
  g1.b = static_cast<const uint8_t*>(a->w1);
  g1.b_scale = a->w1_sf;
  g1.c = nullptr;
  g1.counts = at<int32_t>(ws, l.counts_offset);
  g1.offsets = at<int32_t>(ws, l.offsets_offset);
  g1.num_experts = a->num_experts;
  g1.n = 2 * a->intermediate;
  g1.k = a->hidden;
  g1.engine = engine;
  g1.sw.enabled = 1;
  g1.sw.inter = a->intermediate;
  g1.sw.row_weight = at<float>(ws, l.row_weight_offset);
  g1.sw.y = at<uint16_t>(ws, l.y_offset);
  g1.sw.has_clamp = isfinite(a->activation_clamp) ? 1 : 0;
  g1.sw.clamp = a->activation_clamp;
  g1.sched = at<int32_t>(ws, l.sched_offset);
  if (route_in_gemm1) {
    g1.route_in_kernel = 1;
    g1.route = forward_route_args(a, l);
  }
  if (route_small_in_gemm1) g1.route = forward_route_args(a, l);
  // Whole-layer calls on the WIDE GEMM1: its workgroups out of tiles write the zero y rows of
  // tokens without a valid routed slot, and the combine skips them. The routing launch of the
  // same call zeroes the claim counter (also when it returns at once).
  const bool zero_fill = runs(MMOE_STAGE_ROUTE) && !route_in_gemm1 && runs(MMOE_STAGE_COMBINE) &&
                         a->hidden % 8 == 0 && mmoe::gemm_wide_selected(g1, max_rows);
  int32_t* zfill_claim = at<int32_t>(ws, l.sched_offset) + mmoe::kZeroFillClaim;
  if (zero_fill) {
    g1.zf.y = static_cast<uint16_t*>(a->y);
    g1.zf.claim = zfill_claim;
    g1.zf.idle = zfill_claim + 1;
    g1.zf.output_index = at<int32_t>(ws, l.output_index_offset);
    g1.zf.runtime_tokens = a->runtime_num_tokens;
    g1.zf.host_tokens = a->num_tokens;
    g1.zf.topk = a->num_topk;
    g1.zf.hidden = a->hidden;
  }

  mmoe::GemmArgs g2 = g1;
  memset(&g2.sw, 0, sizeof(g2.sw));
  if (zero_fill) g2.zf.idle = zfill_claim + 2;  // (the same chunks, claimed on from GEMM1's)
  g2.route_in_kernel = 0;
  g2.a = at<uint8_t>(ws, l.act_offset);
  g2.row_token = nullptr;
  g2.a_scale = at<float>(ws, l.act_scale_offset);
  g2.lda = a->intermediate;
  g2.b = static_cast<const uint8_t*>(a->w2);
  g2.b_scale = a->w2_sf;
  g2.c = at<uint16_t>(ws, l.part_offset);
  g2.n = a->hidden;
  g2.k = a->intermediate;
  g2.sched = at<int32_t>(ws, l.sched_offset) + mmoe::kSchedInts;
  // Prefill: rows whose token has a single routed slot leave the WIDE GEMM2 straight into y
  // (the combine's one-term sum), so the combine neither reads nor writes them. The requant
  // builds the row table and sets meta[2]; GEMM2 and the combine follow meta[2] on the device,
  // so the stages behave the same in one call or in several.
  const bool direct = mmoe::gemm_wide_selected(g2, max_rows) && l.row_capacity >= max_rows;
  int32_t* direct_flag = at<int32_t>(ws, l.meta_offset) + 2;
  mmoe::RowDest dest;
  memset(&dest, 0, sizeof(dest));
  dest.meta_flag = direct_flag;
  if (direct) {
    dest.row_dest = at<int32_t>(ws, l.row_dest_offset);
    dest.row_token = at<int32_t>(ws, l.row_token_offset);
    dest.output_index = at<int32_t>(ws, l.output_index_offset);
    dest.topk = a->num_topk;
    g2.row_dest = dest.row_dest;
    g2.y_direct = static_cast<uint16_t*>(a->y);
    g2.direct_flag = direct_flag;
  }

  // Decode (GEMM1 routes in-kernel): GEMM1, the requant, GEMM2 and (when the call includes it)
  // the combine in one launch, each group of rows going on to GEMM2 as soon as its GEMM1 items
  // are done, each token combined as soon as its experts' GEMM2 items are. Its last workgroup
  // sets its counters back to zero.
  bool combined = false;
  if (route_in_gemm1 && runs(MMOE_STAGE_REQUANT) && runs(MMOE_STAGE_GEMM2) && !direct &&
      mmoe::decode_pipeline_supported(g1, g2, cus)) {
    mmoe::PipeArgs p;
    memset(&p, 0, sizeof(p));
    p.g1 = g1;
    p.g1.row_pmax = at<float>(ws, l.pmax_offset);
    p.g2 = g2;
    p.act = at<uint8_t>(ws, l.act_offset);
    p.act_scale = at<float>(ws, l.act_scale_offset);
    p.amax = at<float>(ws, l.amax_offset);
    p.meta = at<int32_t>(ws, l.meta_offset);
    p.direct_flag = direct_flag;
    p.pipe = at<int32_t>(ws, l.pipe_offset);
    p.spin_limit = (a->debug_flags & MMOE_DEBUG_NO_WAIT) != 0 ? 0 : mmoe::kPipeSpinLimit;
    if (runs(MMOE_STAGE_COMBINE) && a->hidden % 8 == 0 && a->hidden <= mmoe::kPipeCombineMaxHidden) {
      p.y = static_cast<uint16_t*>(a->y);
      combined = true;
    }
    mark_stage(MMOE_STAGE_PIPELINE);
    if (mmoe::launch_decode_pipeline(p, cus, s) != hipSuccess) return MMOE_ERR_HIP;
  } else {
    // Eager calls whose bound selects WIDE by a small margin: the routing's largest expert row
    // count (meta[4]) chooses between WIDE and the 8-wave kernels on the device as well
    // (gemm_eager_dual; these calls never route in GEMM1).
    const bool eager_dual = a->runtime_num_tokens == nullptr && mmoe::gemm_eager_dual(g1, max_rows);
    const int32_t* dual_rows = eager_dual ? at<int32_t>(ws, l.meta_offset) + 4 : rows_on_device;
    const int dual_min = eager_dual ? mmoe::gemm_eager_dual_min_largest()
                                    : mmoe::gemm_wide_min_rows(a->num_experts);
    mark_stage(MMOE_STAGE_GEMM1);
    if (runs(MMOE_STAGE_GEMM1) &&
        mmoe::launch_grouped_gemm(g1, max_rows, cus, s, dual_rows, route_small_in_gemm1, dual_min) != hipSuccess)
      return MMOE_ERR_HIP;
    // (after a dual GEMM1 launch the requant finds out on the device which GEMM1 ran: the
    // direct-write table goes with the WIDE GEMMs only)
    const bool wide1 = mmoe::gemm_wide_selected(g1, max_rows);
    const bool dual1 = wide1 && dual_rows != nullptr;
    mark_stage(MMOE_STAGE_REQUANT);
    if (runs(MMOE_STAGE_REQUANT) &&
        mmoe::launch_requant(at<uint16_t>(ws, l.y_offset), wide1, at<float>(ws, l.amax_offset),
                             at<int32_t>(ws, l.meta_offset), at<uint8_t>(ws, l.act_offset),
                             at<float>(ws, l.act_scale_offset), max_rows, a->intermediate, dest,
                             cus, s, dual1 ? dual_rows : nullptr, dual_min) != hipSuccess)
      return MMOE_ERR_HIP;
    mark_stage(MMOE_STAGE_GEMM2);
    if (runs(MMOE_STAGE_GEMM2) &&
        mmoe::launch_grouped_gemm(g2, max_rows, cus, s, dual_rows, false, dual_min) != hipSuccess)
      return MMOE_ERR_HIP;
  }

  if (runs(MMOE_STAGE_COMBINE) && !combined) {
    mark_stage(MMOE_STAGE_COMBINE);
    mmoe::CombineArgs c;
    memset(&c, 0, sizeof(c));
    c.y = static_cast<uint16_t*>(a->y);
    c.part = at<uint16_t>(ws, l.part_offset);
    c.output_index = at<int32_t>(ws, l.output_index_offset);
    c.runtime_tokens = a->runtime_num_tokens;
    c.host_tokens = a->num_tokens;
    c.topk = a->num_topk;
    c.hidden = a->hidden;
    c.skip_single = direct_flag;
    if (zero_fill) c.zfill_claim = zfill_claim;
    if (mmoe::launch_combine(c, cus, s) != hipSuccess) return MMOE_ERR_HIP;
  }
  return MMOE_OK;
}

static_assert(MMOE_PIPE_INTS == mmoe::kPipeInts, "the header's pipeline counter count");
static_assert(MMOE_PIPE_INTS * 4 % 256 == 0 && MMOE_SCRATCH_STATUS_OFFSET == MMOE_PIPE_INTS * 4 + 12,
              "meta follows the pipeline counters directly (the status offset of every layout)");

int mmoe_scratch_status(const void* route_scratch, int32_t* out, void* stream) {
  if (out == nullptr) return MMOE_ERR_NULL_POINTER;
  const void* base = route_scratch;
  if (base == nullptr) {  // the static scratch of mmoe_forward_static on this device
    void* p = nullptr;
    const int st = static_scratch_address(&p);
    if (st != MMOE_OK) return st;
    base = p;
  }
  const void* src = static_cast<const uint8_t*>(base) + MMOE_SCRATCH_STATUS_OFFSET;
  return hipMemcpyAsync(out, src, sizeof(int32_t), hipMemcpyDefault,
                        static_cast<hipStream_t>(stream)) == hipSuccess
             ? MMOE_OK
             : MMOE_ERR_HIP;
}

int mmoe_forward(const mmoe_forward_args* a, void* stream) {
  return mmoe_forward_stages(a, MMOE_STAGE_ROUTE, MMOE_STAGE_COMBINE, stream);
}

int mmoe_forward_profile(const mmoe_forward_args* a, void* stream, void* const* events,
                         int capacity, int32_t* stages, int32_t* num_launches) {
  if (capacity < 0 || (capacity > 0 && events == nullptr)) return MMOE_ERR_ARGUMENT;
  mmoe::LaunchTimer timer;
  timer.events = reinterpret_cast<hipEvent_t const*>(events);
  timer.stages = stages;
  timer.capacity = capacity;
  timer.count = 0;
  timer.stage = MMOE_STAGE_ROUTE;
  mmoe::LaunchTimer*& slot = mmoe::launch_timer();
  mmoe::LaunchTimer* const outer = slot;
  slot = &timer;
  const int st = mmoe_forward_stages(a, MMOE_STAGE_ROUTE, MMOE_STAGE_COMBINE, stream);
  slot = outer;
  if (num_launches != nullptr) *num_launches = timer.count;
  return st;
}

int mmoe_forward_static(const mmoe_forward_args* args, void* stream) {
  if (args == nullptr) return MMOE_ERR_NULL_POINTER;
  mmoe_forward_args a = *args;
  const int st = check_common(1, a.num_experts, a.num_max_tokens, a.num_topk, a.hidden,
                              a.intermediate);
  if (st != MMOE_OK) return st;
  mmoe_scratch_layout l;
  plan_scratch(1, a.num_experts, a.num_max_tokens, a.num_topk, a.hidden, a.intermediate, &l);
  if (l.total_bytes > MMOE_STATIC_SCRATCH_BYTES) return MMOE_ERR_STATIC_SCRATCH;
  // the same launch sequence as mmoe_forward, on the static scratch of this device: nothing
  // is allocated. The array starts zero-filled, and every call leaves the only counters that
  // must be zero when a call starts (the decode pipeline's) at zero.
  void* p = nullptr;
  const int sst = static_scratch_address(&p);
  if (sst != MMOE_OK) return sst;
  a.route_scratch = p;
  a.route_scratch_bytes = MMOE_STATIC_SCRATCH_BYTES;
  return mmoe_forward_stages(&a, MMOE_STAGE_ROUTE, MMOE_STAGE_COMBINE, stream);
}

int mmoe_deepep_preprocess_workspace_bytes(int recv_rows, int topk, int num_experts,
                                           int total_rows, int64_t* out_bytes) {
  if (out_bytes == nullptr) return MMOE_ERR_NULL_POINTER;
  if (recv_rows < 0 || topk <= 0 || num_experts <= 0 || num_experts > mmoe::kMaxExperts ||
      total_rows < 0)
    return MMOE_ERR_ARGUMENT;
  const int64_t tasks = static_cast<int64_t>(recv_rows) * topk;
  int64_t off = 0;
  off = align_up(off + num_experts * 4, 256);            // counts
  off = align_up(off + (num_experts + 1) * 4, 256);      // offsets
  off = align_up(off + 16 * 4, 256);                     // meta
  off = align_up(off + mmoe::route_count_ints(tasks, num_experts) * 4, 256);  // chunk, wave counts
  off = align_up(off + (total_rows > 0 ? total_rows : 1) * 4, 256);  // row_token
  *out_bytes = off;
  return MMOE_OK;
}

int mmoe_deepep_preprocess_channelwise(void* grouped_x, float* grouped_x_scale,
                                       float* route_weights, int32_t* m_indices,
                                       int32_t* output_index, const void* recv_x,
                                       const float* recv_x_scale, const void* recv_topk_ids,
                                       const float* recv_topk_weights,
                                       const int32_t* num_recv_tokens_per_expert,
                                       int total_rows, int recv_rows, int topk, int hidden,
                                       int num_experts, int topk_ids_i64, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  int64_t need = 0;
  int st = mmoe_deepep_preprocess_workspace_bytes(recv_rows, topk, num_experts, total_rows, &need);
  if (st != MMOE_OK) return st;
  if (workspace_bytes < need) return MMOE_ERR_SCRATCH_SMALL;
  if (hidden <= 0) return MMOE_ERR_HIDDEN_SIZES;
  const int64_t tasks = static_cast<int64_t>(recv_rows) * topk;
  if (tasks == 0) return MMOE_OK;
  if (grouped_x == nullptr || grouped_x_scale == nullptr || route_weights == nullptr ||
      m_indices == nullptr || output_index == nullptr || recv_x == nullptr ||
      recv_x_scale == nullptr || recv_topk_ids == nullptr || recv_topk_weights == nullptr ||
      num_recv_tokens_per_expert == nullptr || workspace == nullptr)
    return MMOE_ERR_NULL_POINTER;
  const int64_t chunks = (tasks + mmoe::kRouteChunk - 1) / mmoe::kRouteChunk;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t a0 = off;
    off = align_up(off + bytes, 256);
    return a0;
  };
  mmoe::RouteArgs r;
  memset(&r, 0, sizeof(r));
  r.counts = at<int32_t>(workspace, take(num_experts * 4));
  r.offsets = at<int32_t>(workspace, take((num_experts + 1) * 4));
  r.meta = at<int32_t>(workspace, take(16 * 4));
  r.chunk_counts = at<int32_t>(workspace, take(mmoe::route_count_ints(tasks, num_experts) * 4));
  r.wave_counts = r.chunk_counts + (chunks > 0 ? chunks : 1) * num_experts;
  r.row_token = at<int32_t>(workspace, take((total_rows > 0 ? total_rows : 1) * 4));
  r.topk_idx = recv_topk_ids;
  r.idx_i64 = topk_ids_i64 ? 1 : 0;
  r.topk_w = recv_topk_weights;
  r.host_tokens = recv_rows;
  r.topk = topk;
  r.num_experts = num_experts;
  r.check_weight = 0;
  r.row_cap = total_rows;
  r.given_counts = num_recv_tokens_per_expert;
  r.output_index = output_index;
  r.row_weight = route_weights;
  r.m_indices = m_indices;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mmoe::launch_route(r, tasks, s) != hipSuccess) return MMOE_ERR_HIP;
  if (mmoe::launch_gather_tasks(static_cast<uint8_t*>(grouped_x), grouped_x_scale,
                                static_cast<const uint8_t*>(recv_x), recv_x_scale, output_index,
                                tasks, topk, hidden, s) != hipSuccess)
    return MMOE_ERR_HIP;
  return MMOE_OK;
}

int mmoe_deepep_postprocess_channelwise(void* recv_y, const void* l2_out,
                                        const void* recv_topk_ids,
                                        const float* recv_topk_weights,
                                        const int32_t* output_index, int recv_rows, int topk,
                                        int hidden, int topk_ids_i64, int apply_topk_weights,
                                        void* stream) {
  if (recv_rows < 0 || topk <= 0 || topk > kMaxTopk || hidden <= 0) return MMOE_ERR_ARGUMENT;
  if (recv_rows == 0) return MMOE_OK;
  if (recv_y == nullptr || l2_out == nullptr || recv_topk_ids == nullptr ||
      recv_topk_weights == nullptr || output_index == nullptr)
    return MMOE_ERR_NULL_POINTER;
  int cus = 0;
  const int st = device_cus(&cus);
  if (st != MMOE_OK) return st;
  mmoe::CombineArgs c;
  memset(&c, 0, sizeof(c));
  c.y = static_cast<uint16_t*>(recv_y);
  c.part = static_cast<const uint16_t*>(l2_out);
  c.output_index = output_index;
  c.topk_ids = recv_topk_ids;
  c.ids_i64 = topk_ids_i64 ? 1 : 0;
  c.topk_w = recv_topk_weights;
  c.apply_weights = apply_topk_weights ? 1 : 0;
  c.host_tokens = recv_rows;
  c.topk = topk;
  c.hidden = hidden;
  return mmoe::launch_combine(c, cus, static_cast<hipStream_t>(stream)) == hipSuccess
             ? MMOE_OK
             : MMOE_ERR_HIP;
}

int mmoe_cast_fp8_channelwise(void* out_fp8, float* out_scale, const void* x_bf16, int64_t rows,
                              int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return MMOE_ERR_ARGUMENT;
  if (rows == 0) return MMOE_OK;
  if (out_fp8 == nullptr || out_scale == nullptr || x_bf16 == nullptr) return MMOE_ERR_NULL_POINTER;
  return mmoe::launch_cast_fp8_channelwise(static_cast<uint8_t*>(out_fp8), out_scale,
                                           static_cast<const uint16_t*>(x_bf16), rows, cols,
                                           static_cast<hipStream_t>(stream)) == hipSuccess
             ? MMOE_OK
             : MMOE_ERR_HIP;
}

int mmoe_marlin_pack(void* out, const void* in, int64_t groups, int64_t rows, int64_t k,
                     void* stream) {
  if (groups < 0 || rows < 0 || k < 0) return MMOE_ERR_ARGUMENT;
  if (rows % 16 || k % 16) return MMOE_ERR_MARLIN_DIVISIBLE;
  if (groups * rows * k == 0) return MMOE_OK;
  if (out == nullptr || in == nullptr) return MMOE_ERR_NULL_POINTER;
  return mmoe::launch_marlin_pack(static_cast<uint8_t*>(out), static_cast<const uint8_t*>(in),
                                  groups, rows, k, static_cast<hipStream_t>(stream)) == hipSuccess
             ? MMOE_OK
             : MMOE_ERR_HIP;
}

int mmoe_debug_f32_to_e4m3(uint8_t* out, const float* in, int64_t n, void* stream) {
  if (n < 0) return MMOE_ERR_ARGUMENT;
  if (n == 0) return MMOE_OK;
  if (out == nullptr || in == nullptr) return MMOE_ERR_NULL_POINTER;
  return mmoe::launch_f32_to_e4m3(out, in, n, static_cast<hipStream_t>(stream)) == hipSuccess
             ? MMOE_OK
             : MMOE_ERR_HIP;
}

}  // extern "C"
