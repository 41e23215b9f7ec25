/*
 * megamoe_hip.h -- C ABI of the MI355X (gfx950) FP8 W8A8 channelwise Mega MoE forward.
 *
 * Plain C: pointers, sizes and status codes only. Every device pointer is a HIP device
 * address; `stream` is a hipStream_t passed as void* (NULL = the default stream). All calls
 * that take a stream are asynchronous and stream-ordered: they never synchronise the host,
 * never allocate device memory and keep no per-call global state.
 *
 * Each entry point names the reference interface it replaces (paths relative to the
 * yuguo-Jack/DeepGEMM tree). The Python mirror in deepgemm_amd/megamoe binds these with ctypes.
 *
 * Tensor layouts (identical to the reference's):
 *   x            e4m3fn  [S_max, H]              row-major activations (per-token scale)
 *   x_sf         f32     [S_max]
 *   topk_idx     int64   [S_max, K]              expert id, <0 or >=E = not routed here
 *   topk_weights f32     [S_max, K]              0 = not routed (reference rule)
 *   w1           e4m3fn  [E, 2I/16, H*16]        Marlin nt_kpack2 (gate rows [0,I), up rows [I,2I))
 *   w1_sf        f32     [E, 2I]
 *   w2           e4m3fn  [E, H/16, I*16]         Marlin nt_kpack2
 *   w2_sf        f32     [E, H]
 *   y            bf16    [S, H]                  written in place
 *   stats        int32   [E]                     optional, accumulated (+= routed rows)
 */
#ifndef MEGAMOE_HIP_H_
#define MEGAMOE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: 0 = OK, negative = the reference check that failed ---- */
#define MMOE_OK 0
#define MMOE_ERR_NULL_POINTER (-1)       /* a required pointer is NULL */
#define MMOE_ERR_NUM_RANKS (-2)          /* "num_ranks must be positive" / single-GPU build */
#define MMOE_ERR_EXPERTS_DIVISIBLE (-3)  /* "num_experts must be divisible by num_ranks" */
#define MMOE_ERR_HIDDEN_SIZES (-4)       /* "hidden sizes must be positive" */
#define MMOE_ERR_MARLIN_DIVISIBLE (-5)   /* "... Marlin weights require rows and K divisible by 16" */
#define MMOE_ERR_TOO_MANY_TOKENS (-6)    /* "too many tokens" */
#define MMOE_ERR_SYM_BUFFER_SMALL (-7)   /* "sym_buffer is too small ..." */
#define MMOE_ERR_SCRATCH_SMALL (-8)      /* "route_scratch is too small ..." */
#define MMOE_ERR_UNSUPPORTED_SHAPE (-9)  /* shape outside what the gfx950 kernels tile */
#define MMOE_ERR_TOPK (-10)              /* top-k out of range */
#define MMOE_ERR_SCHEDULE (-11)          /* unknown schedule override */
#define MMOE_ERR_HIP (-12)               /* a HIP runtime call failed (launch error) */
#define MMOE_ERR_NO_DEVICE (-13)         /* no usable HIP device / not gfx950 */
#define MMOE_ERR_ARGUMENT (-14)          /* other invalid argument */
#define MMOE_ERR_STATIC_SCRATCH (-15)    /* mmoe_forward_static: call exceeds the static scratch */

/* Schedule of mmoe_forward (the reference's MEGAMOE_DCU_USE_LARGE_OPT_3STAGE auto/off/force).
 * The grouped GEMMs have two tile engines; AUTO picks one per expert on the device from its
 * routed row count (<= 128 rows: weight-streaming engine; more: 256x256 MFMA tile engine). When
 * every expert has many rows (S*K > 8192 and at least 256 rows per expert on average), AUTO
 * and STAGED run both GEMMs on a 4-wave 256x256 kernel instead. */
#define MMOE_SCHEDULE_AUTO 0       /* per-expert choice on the device */
#define MMOE_SCHEDULE_PERSISTENT 1 /* streaming engine for every expert (HBM-bound decode) */
#define MMOE_SCHEDULE_STAGED 2     /* tile engine for every expert (MFMA-bound prefill) */

/* Byte layout of the per-GPU input buffer (the reference's sym_buffer).
 * Replaces get_symm_buffer_size_for_mega_moe and its slicer,
 * csrc/apis/mega_dcu.hpp:93-154 (offsets in bytes from the buffer base). */
typedef struct mmoe_symm_layout {
  int64_t total_bytes;
  int64_t runtime_num_tokens_offset; /* int32 [1] (cuda_graph_num_tokens) */
  int64_t x_offset;                  /* e4m3 [S_max, H] */
  int64_t x_sf_offset;               /* f32 [S_max] */
  int64_t topk_idx_offset;           /* int64 [S_max, K] */
  int64_t topk_weights_offset;       /* f32 [S_max, K] */
} mmoe_symm_layout;

/* Byte offsets of the intermediates inside route_scratch (debug / stage-parity views).
 * Replaces the reference's route-scratch carving, megamoe/large_opt.py:153-251 and
 * deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:144-265. */
typedef struct mmoe_scratch_layout {
  int64_t total_bytes;
  int64_t row_capacity;        /* rows reserved for routed (token, expert) pairs */
  int64_t num_chunks;          /* routing chunks of MMOE_ROUTE_CHUNK tasks */
  int64_t counts_offset;       /* int32 [E]   rows per local expert */
  int64_t offsets_offset;      /* int32 [E+1] first row of each expert (exclusive scan) */
  int64_t meta_offset;         /* int32 [16]  [0] = total routed rows R; [1] = 1: GEMM1 ran on
                                  the WIDE kernel; [2] = 1: GEMM2 wrote
                                  the rows of single-slot tokens straight to y (row_dest);
                                  [3] = the call's status (bounded waits of the decode pipeline
                                  that ran out; 0 = y is valid; MMOE_SCRATCH_STATUS_OFFSET);
                                  [4] = the largest expert's row count (routing launches) */
  int64_t chunk_counts_offset; /* int32 [num_chunks, E] per-chunk counts, then
                                  [num_chunks, 16, E] per-wave counts (routing) */
  int64_t output_index_offset; /* int32 [S_max, K]  row of (token, slot) or -1 */
  int64_t row_token_offset;    /* int32 [rows] source token of each routed row */
  int64_t row_weight_offset;   /* f32   [rows] top-k weight of each routed row */
  int64_t m_indices_offset;    /* int32 [rows] local expert of each routed row */
  int64_t act_scale_offset;    /* f32   [rows] per-row FP8 scale of the SwiGLU output */
  int64_t amax_offset;         /* f32   [rows] max |y| per row (written by the requant stage) */
  int64_t y_offset;            /* bf16  [rows, I]  SwiGLU x weight output of GEMM1 */
  int64_t act_offset;          /* e4m3  [rows, I]  requantised SwiGLU output */
  int64_t part_offset;         /* bf16  [rows, H]  per-row GEMM2 output (combine partials);
                                  in a prefill call (WIDE GEMMs) the rows of tokens with a
                                  single routed slot go straight to y instead (row_dest) */
  int64_t row_dest_offset;     /* int32 [rows] token of a row written straight to y, else -1
                                  (valid after a call that used it) */
  int64_t sched_offset;        /* int32 [2, 16] work-claim counters of the prefill GEMM kernels
                                  (GEMM1, GEMM2): zeroed by the routing stage, left at zero by
                                  the GEMMs themselves */
  int64_t pipe_offset;         /* int32 [MMOE_PIPE_INTS] counters of the one-launch decode
                                  pipeline (GEMM1 + requant + GEMM2 + combine), always at offset
                                  0 whatever the shape: they must be zero when a call starts --
                                  zero when the scratch is new (allocate it zero-filled), and
                                  left zero by every call, so a scratch may serve calls of any
                                  shape in turn */
  int64_t pmax_offset;         /* f32   [min(rows, 8192), 2I/64] the decode pipeline's per-row
                                  max |y| of each 64-column block of GEMM1's output */
} mmoe_scratch_layout;

#define MMOE_ROUTE_CHUNK 1024
#define MMOE_PIPE_INTS 4928
/* Byte offset of meta[3] (the status of the last call) in every route_scratch: the pipeline
 * counters (MMOE_PIPE_INTS ints at offset 0) and then meta. */
#define MMOE_SCRATCH_STATUS_OFFSET (MMOE_PIPE_INTS * 4 + 3 * 4)

/* Bits of mmoe_forward_args.debug_flags (0 in production). */
#define MMOE_DEBUG_NO_WAIT 1 /* every bounded wait of the decode pipeline gives up at its first
                                poll: the launch still ends, and the call's status reports the
                                waits (tests of the error path) */

/* Arguments of one layer call. Replaces the argument list of fp8_mega_moe_impl,
 * csrc/apis/mega_dcu.hpp:338-354, and of
 * launch_mega_moe_multirank_persistent_hip_w8a8_channelwise, csrc/apis/mega_dcu.hpp:41-55. */
typedef struct mmoe_forward_args {
  void* y;                           /* bf16 [num_tokens, H] out */
  const void* x;                     /* e4m3 [S_max, H] */
  const float* x_sf;                 /* f32 [S_max] */
  const int64_t* topk_idx;           /* int64 [S_max, K] */
  const float* topk_weights;         /* f32 [S_max, K] */
  const void* w1;                    /* e4m3 Marlin [E, 2I/16, H*16] */
  const float* w1_sf;                /* f32 [E, 2I] */
  const void* w2;                    /* e4m3 Marlin [E, H/16, I*16] */
  const float* w2_sf;                /* f32 [E, H] */
  int32_t* stats;                    /* int32 [E] or NULL (accumulated) */
  void* route_scratch;               /* device workspace, >= mmoe_route_scratch_bytes() */
  int64_t route_scratch_bytes;
  int64_t sym_buffer_bytes;          /* size of the buffer x/x_sf/topk_* live in (checked) */
  const int32_t* runtime_num_tokens; /* device int32 [1] or NULL: tokens read at run time */
  int32_t num_tokens;                /* rows of y */
  int32_t num_max_tokens;            /* S_max (capacity of the input buffer) */
  int32_t num_experts;               /* E local experts */
  int32_t num_topk;                  /* K */
  int32_t hidden;                    /* H */
  int32_t intermediate;              /* I */
  float activation_clamp;            /* +inf = no clamp (reference: activation_clamp=None) */
  int32_t schedule;                  /* MMOE_SCHEDULE_* */
  int32_t debug_flags;               /* 0, or MMOE_DEBUG_* bits (tests only) */
} mmoe_forward_args;

/* get_token_alignment_for_mega_moe, csrc/apis/mega_dcu.hpp:24-26 (kTokenAlignment,
 * deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:9). */
int mmoe_token_alignment(void);

/* get_symm_buffer_size_for_mega_moe, csrc/apis/mega_dcu.hpp:93-154. */
int mmoe_symm_buffer_layout(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                            int hidden, int intermediate, mmoe_symm_layout* out);

/* get_mega_moe_route_scratch_size_for_mega_moe, csrc/apis/mega_dcu.hpp:156-169. */
int mmoe_route_scratch_bytes(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                             int hidden, int intermediate, int64_t* out_bytes);

/* Offsets of the intermediates inside route_scratch (same arguments as above). */
int mmoe_route_scratch_layout(int num_ranks, int num_experts, int num_max_tokens, int num_topk,
                              int hidden, int intermediate, mmoe_scratch_layout* out);

/* get_mega_moe_hip_build_config, csrc/apis/mega_dcu.hpp:28-39; returns a static JSON string. */
const char* mmoe_build_config(void);

/* Human-readable text of a status code. */
const char* mmoe_status_string(int status);

/* The layer: fp8_mega_moe / fp8_mega_moe_with_graph_tokens,
 * csrc/apis/mega_dcu.hpp:338-518 -> csrc/kernels/mega_moe_fused_hip.cu:72-121 and the staged
 * path megamoe/large_opt.py:367-508. Routing -> GEMM1 with fused SwiGLU -> requant -> GEMM2
 * -> combine.
 * Precondition: the first MMOE_PIPE_INTS * 4 bytes of route_scratch are zero when the call
 * starts. Allocate route_scratch zero-filled once; every call leaves those bytes zero again
 * (whatever its shape), so nothing needs clearing between calls. Calls that overlap on one
 * route_scratch race.
 * The return code covers validation and launch errors only. At decode sizes (S*K <= 8192 on
 * the 256-CU MI355X) the layer is one persistent launch whose workgroups hand rows to each other
 * through bounded waits: it needs the whole GPU, and a wait that runs out (another kernel
 * holding CUs for longer than the bound) leaves a wrong y. The launch still ends, and the call's
 * status (mmoe_scratch_status) is nonzero then. */
int mmoe_forward(const mmoe_forward_args* args, void* stream);

/* Status of the last mmoe_forward / mmoe_forward_static call on route_scratch (NULL: the static
 * scratch of the current device): enqueues on `stream` a 4-byte copy of it to *out (device
 * memory, or pinned host memory read after the stream has reached this point). 0: that call's
 * y is valid; > 0: the number of bounded waits of its decode pipeline that ran out (y is not
 * valid). No counterpart in the reference, whose persistent kernel waits for its L2 queue
 * without a bound (deep_gemm/include/deep_gemm/scheduler/mega_moe_dcu.cuh:52-53) and aborts the
 * kernel when a barrier times out (deep_gemm/include/deep_gemm/comm/mega_moe_dcu.cuh:76-90,
 * :104-113); it is for callers that must detect a wait that ran out. */
int mmoe_scratch_status(const void* route_scratch, int32_t* out, void* stream);

/* Allocation-free variant of mmoe_forward. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The caller passes inputs and outputs as for mmoe_forward;
 * args->route_scratch and args->route_scratch_bytes are ignored. The scratch is instead a
 * static device array of MMOE_STATIC_SCRATCH_BYTES that the library holds on each GPU it runs
 * on until the process ends: calls whose mmoe_route_scratch_bytes() (for their num_max_tokens)
 * exceeds it return MMOE_ERR_STATIC_SCRATCH (128 MiB covers a token capacity of 1488 at
 * E = 32, H = 4096, I = 2048, top-6). Nothing is allocated on any call (no hipMalloc, no
 * hipFree, no allocating library routine). Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other host threads) race and must be
 * serialised by the caller. Results are bitwise those of mmoe_forward. */
#define MMOE_STATIC_SCRATCH_BYTES (128ll << 20)
int mmoe_forward_static(const mmoe_forward_args* args, void* stream);

/* Stages of mmoe_forward, in order; each reads what the earlier ones left in route_scratch. */
#define MMOE_STAGE_ROUTE 0   /* counts, offsets, output_index, per-row tables, stats */
#define MMOE_STAGE_GEMM1 1   /* gate||up GEMM + SwiGLU x weight -> y bf16 [R, I] */
#define MMOE_STAGE_REQUANT 2 /* row max |y| -> amax [R], act e4m3 [R, I], act_scale [R];
                                row_dest, meta[2] */
#define MMOE_STAGE_GEMM2 3   /* part bf16 [R, H]; with meta[2] = 1 the rows of single-slot
                                tokens go straight to y */
#define MMOE_STAGE_COMBINE 4 /* y (tokens written by GEMM2 are left as they are) */

/* Runs stages [first_stage, last_stage] of mmoe_forward (mmoe_forward = stages 0..4). Lets a
 * profiler bracket each kernel with events and lets tests check each stage on its own. The
 * reference runs the same stages as K1/K2/K3 (megamoe/large_opt.py:367-508). */
int mmoe_forward_stages(const mmoe_forward_args* args, int first_stage, int last_stage,
                        void* stream);

#define MMOE_STAGE_PIPELINE 5 /* (mmoe_forward_profile) the one-launch decode pipeline: stages 0-4 */

/* mmoe_forward with each kernel launch timed inside the whole layer call: launch i (launch
 * order, i < capacity) goes out through hipExtLaunchKernel with events[2i] as its start and
 * events[2i+1] as its stop event, which take the dispatch's own timestamps (the kernel's duration
 * as a kernel trace reads it, and no event marker between the layer's kernels); stages[i] (may be
 * NULL) = the MMOE_STAGE_* of launch i; *num_launches (may be NULL) = the call's launches (those
 * past capacity run untimed). The events are hipEvent_t made by the caller; read them
 * (hipEventElapsedTime) once the stream has passed them. Asynchronous like mmoe_forward, with the
 * same results. For measurement only; it replaces the reference harness's timing of each call
 * between two stream events (tests/test_mega_moe_dcu.py:326-341). */
int mmoe_forward_profile(const mmoe_forward_args* args, void* stream, void* const* events,
                         int capacity, int32_t* stages, int32_t* num_launches);

/* Routing only (counts, offsets, output_index, row_token, row_weight, m_indices, stats) into
 * route_scratch: the route stage of mmoe_forward exposed for stage parity. The reference
 * computes the same in its route scan, deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:316-425,
 * and in k1_count/build/emit, megamoe/dcu_megamoe_large_opt/K1_fused/k1_fused_ext.cu:254-455. */
int mmoe_route(const mmoe_forward_args* args, void* stream);

/* deepep_deepgemm_preprocess_channelwise, csrc/apis/mega_dcu.hpp:222-292 with
 * csrc/kernels/mega_moe_baseline_hip.cu:37-96. Expert-contiguous scatter of received rows.
 * Rows of an expert are in ascending (token, slot) order (deterministic). Outputs sized
 * [total_rows, ...]; the caller pre-fills route_weights=0, m_indices=-1 like the reference.
 * topk_ids are int64 when topk_ids_i64 != 0 else int32. `workspace` is device scratch of at
 * least mmoe_deepep_preprocess_workspace_bytes() bytes (the reference's expert_start_loc). */
int mmoe_deepep_preprocess_workspace_bytes(int recv_rows, int topk, int num_experts,
                                           int total_rows, int64_t* out_bytes);
int mmoe_deepep_preprocess_channelwise(void* grouped_x, float* grouped_x_scale,
                                       float* route_weights, int32_t* m_indices,
                                       int32_t* output_index, const void* recv_x,
                                       const float* recv_x_scale, const void* recv_topk_ids,
                                       const float* recv_topk_weights,
                                       const int32_t* num_recv_tokens_per_expert,
                                       int total_rows, int recv_rows, int topk, int hidden,
                                       int num_experts, int topk_ids_i64, void* workspace,
                                       int64_t workspace_bytes, void* stream);

/* deepep_deepgemm_postprocess_channelwise, csrc/apis/mega_dcu.hpp:294-336 with
 * csrc/kernels/mega_moe_baseline_hip.cu:98-127: recv_y[t] = bf16(sum_s l2_out[output_index[t,s]]
 * (x w[t,s] if apply_topk_weights)) over valid slots in slot order. */
int mmoe_deepep_postprocess_channelwise(void* recv_y, const void* l2_out,
                                        const void* recv_topk_ids,
                                        const float* recv_topk_weights,
                                        const int32_t* output_index, int recv_rows, int topk,
                                        int hidden, int topk_ids_i64, int apply_topk_weights,
                                        void* stream);

/* Channelwise FP8 cast of one bf16 matrix [rows, cols] -> e4m3 + f32 per-row scale
 * (scale = max(amax, 1e-4)/448, q = e4m3_rne(x/scale)). The on-device form of
 * cast_to_fp8_channelwise / cast_grouped_weight_to_fp8_channelwise, megamoe/__init__.py:51-78. */
int mmoe_cast_fp8_channelwise(void* out_fp8, float* out_scale, const void* x_bf16, int64_t rows,
                              int64_t cols, void* stream);

/* Marlin nt_kpack2 permute of a grouped e4m3 weight [G, R, K] -> [G, R/16, K*16]:
 * weight8bit_nt_kpack2_marlin, megamoe/__init__.py:81-98 (addressing
 * deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66). */
int mmoe_marlin_pack(void* out, const void* in, int64_t groups, int64_t rows, int64_t k,
                     void* stream);

/* Elementwise f32 -> e4m3fn (saturating RNE after a clip to +-448, the conversion every
 * quantising kernel here uses); exposed so the conversion can be checked exhaustively. */
int mmoe_debug_f32_to_e4m3(uint8_t* out, const float* in, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEGAMOE_HIP_H_ */
