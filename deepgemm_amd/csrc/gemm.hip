// gemm.hip -- grouped FP8 (OCP e4m3) GEMMs of the layer on gfx950 MFMA, over the
// expert-contiguous routed rows.
//
// GEMM1 (gate+up, K = H) gathers its A rows straight from the token matrix through row_token
// (the dispatch "pull" of the reference's K1, megamoe/dcu_megamoe_large_opt/K1_fused/
// k1_fused_ext.cu:479-746), so no grouped copy of x exists:
//   h = bf16(acc * x_sf[token] * w1_sf[e, n])       for the gate and the up column of a channel
// On the 8-wave kernel it fuses the K2 stage (megamoe/dcu_megamoe_large_opt/K2_fused/
// k2_fused_ext.cu:254-377) into its epilogue:
//   y = silu(min(h_g, c)) * clamp(h_u, -c, c) * w    (fp32, left to right)
// (each output tile holds matching gate and up channels, so SwiGLU is elementwise in
// registers); on the WIDE kernel it writes h itself (bf16, the staged K1 output) and the
// requant kernel computes y. The per-row requant (amax = max |y|; a = max(amax, 1e-4);
// act = e4m3(clip(y * 448/a)); act_scale = a/448) needs the whole row and runs as its own small
// kernel: a cross-workgroup hand-off inside GEMM1 would need an agent-scope release per tile,
// which on gfx950 writes back the whole (per-XCD, non-coherent) L2 -- measured 4x slower than
// the kernel boundary.
// GEMM2 (down, K = I) reads act/act_scale and writes the bf16 partial rows for the combine:
//   part[r, n] = bf16((sum_k act[r,k] * w2[e,n,k]) * act_scale[r] * w2_sf[e,n]).
//
// B is the Marlin nt_kpack2 weight (deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66):
// per 16-row tile, each 16-byte k-block of the 16 rows is 256 contiguous bytes.
//
// Two persistent kernels per GEMM; the host picks one (gemm_wide_selected):
//  * the 8-wave kernel (one workgroup per CU) runs two tile engines, each expert's chosen on
//    the device from its routed row count, and can route the tasks itself (decode sizes):
//    - STREAM engine (<= 128 rows on the auto schedule: decode, HBM-bound on the weights).
//      A workgroup tile is (expert, 512 output columns, <= 128 rows: 1, 2 or 4 row tiles of
//      32) over the full K; wave w owns columns
//      [64w, 64w + 64) and streams its weight columns from global memory into a register ring
//      4 steps deep (Marlin gives each lane 16 contiguous k-bytes of one weight row; 16 lanes
//      read 256 contiguous bytes), with no barrier: B never touches LDS. The A rows, the same
//      for the 8 waves, go to LDS once per workgroup in k-chunks of 64 KB loaded as whole
//      128-byte lines, double buffered, one barrier per chunk (1-4 per tile). Loading A per
//      wave in MFMA operand order (32 lines per instruction, re-read by every wave) made the A
//      reads, not the weights, set the pace.
//    - TILE engine (more rows). A 256 x 256 output tile per workgroup, the 8 waves as 2 x 4
//      with 128 x 64 each, K in 128-byte stages through double-buffered LDS (A rows
//      XOR-swizzled, B in Marlin's own 256-byte blocks).
//    Both engines let lane l supply k-bytes [32*(l/32), 32*(l/32)+32) of each 64-k MFMA step
//    for A and B alike and accumulate the 64-k steps in the same order.
//  * the 4-wave WIDE kernel (every expert with many rows: prefill, MFMA-bound): one wave per
//    SIMD with its 256 accumulators in AGPRs, 256 x 256 tiles, weights straight into
//    registers and only A through LDS; described at wide_tile.
#include <algorithm>
#include <atomic>

#include "common.cuh"
#include "kernels.h"
#include "launch.h"
#include "route_wave.cuh"

namespace mmoe {

namespace {

constexpr int kGemmThreads = 512;  // 8 waves, one workgroup per CU
constexpr int kGemmWaves = kGemmThreads / kWave;
constexpr int kMaxGemmExperts = 256;
// STREAM engine
constexpr int kStreamUnit = 64;     // output columns per wave
constexpr int kStreamRows = 64;     // rows of a decode pipeline group
constexpr int kStreamItemRows = 128;  // rows of a STREAM item of the 8-wave GEMM kernel
constexpr int kStreamAutoMaxRows = kStreamItemRows;  // the auto schedule streams experts up to this
constexpr int kStreamDepth = 4;     // 64-k weight steps in flight per wave
constexpr int kAChunk = 65536;      // bytes of one A chunk buffer (32*MT rows x 2048/MT k)
constexpr int kALoads = kAChunk / 1024 / kGemmWaves;  // 16-byte A loads per lane per chunk
// TILE engine: 256 x 256 output tile, BK = 128, the 8 waves as 2 (M) x 4 (N), each wave 128
// rows x 64 columns (4 x 2 MFMA tiles of 32 x 32)
constexpr int kTileBM = 256, kTileBN = 256, kTileBK = 128;
constexpr int kTileWM = 2, kTileWN = 4;
constexpr int kTileStage = (kTileBM + kTileBN) * kTileBK;  // 64 KB: A rows, then B row-tiles
constexpr int kSmemBytes = 2 * kAChunk;  // == 2 * kTileStage

__device__ __forceinline__ v8i make_v8i(const int4& lo, const int4& hi) {
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

__device__ __forceinline__ v16f mfma_fp8(const v8i& a, const v8i& b, const v16f& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ int4 ld16(const uint8_t* p) { return *reinterpret_cast<const int4*>(p); }

// Streaming load for data read exactly once (the STREAM engine's weights): the nontemporal
// hint keeps it from displacing reused lines in L2/MALL; measured 6.85 vs 6.15 TB/s for a
// one-pass read with one 8-wave workgroup per CU.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld16_stream(const uint8_t* p) {
  const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
  return make_int4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Where a GEMM finds the token (gather) and the route weight (SwiGLU) of routed row r: the
// routing tables in global memory, or a workgroup's LDS copy of its rows (in-kernel routing),
// entry r - base.
struct RowSrc {
  const int32_t* tok;
  const float* w;
  int base;
  __device__ __forceinline__ int token(int r) const { return tok[r - base]; }
  __device__ __forceinline__ float weight(int r) const { return w[r - base]; }
};

template <bool kGather>
__device__ __forceinline__ float row_scale(const GemmArgs& g, const RowSrc& rs, int row) {
  return kGather ? g.a_scale[rs.token(row)] : g.a_scale[row];
}

template <bool kGather>
__device__ __forceinline__ const uint8_t* a_row_ptr(const GemmArgs& g, const RowSrc& rs, int row) {
  const int64_t src = kGather ? static_cast<int64_t>(rs.token(row)) : row;
  return g.a + src * g.lda;
}

// Weight row (output column of B) of column tile `ct` (32 columns) of n-block `nb`. With the
// SwiGLU epilogue, tile nb holds gate channels [nb*W, nb*W+W) then the same up channels
// (rows I + ...), W = columns per tile / 2.
template <bool kSwiglu>
__device__ __forceinline__ int weight_row(const GemmArgs& g, int nb, int tile_cols, int col) {
  if (!kSwiglu) return nb * tile_cols + col;
  const int half = tile_cols / 2;
  return col < half ? nb * half + col : g.sw.inter + nb * half + (col - half);
}

// SwiGLU of one (row, channel): h rounded to bf16 exactly like the staged K1 output.
__device__ __forceinline__ float swiglu_value(const GemmArgs& g, float gacc, float uacc, float xs,
                                              float wsg, float wsu, float route_w) {
  return swiglu_weighted(bf16_round(gacc * xs * wsg), bf16_round(uacc * xs * wsu), route_w,
                         g.sw.has_clamp, g.sw.clamp);
}

// Thread index for an engine body, opaque to the optimizer: values derived from it are computed
// inside the body instead of being hoisted out of the persistent item loop, where the
// invariants of every engine variant would stay live at once and crowd out the ring.
__device__ __forceinline__ int opaque_tid() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}

// ------------------------------------------------------------------ epilogue
// Per-tile scales: row r's A scale (its token's, when gathering) and route weight (SwiGLU), and
// each lane's weight-row scales (GEMM2: its column in both 32-column tiles; SwiGLU: its gate and
// up channel). They are loaded into registers at the start of an item and written into a static
// LDS table just before the barrier that completes the item's first A chunk (or stage): the A
// loads issued after them have landed by then, so that costs no wait of its own, and the
// epilogue reads LDS instead of memory. (Loaded before a tile's last MFMAs instead, the compiler
// sank the loads into the epilogue: a memory round trip after the last MFMA, then a full vmcnt
// wait behind the first output stores.)
struct TileTables {
  float xs[kTileBM];               // row scale of tile row r
  float rw[kTileBM];               // route weight of tile row r (SwiGLU)
  float bs[kGemmWaves][2][kWave];  // wave w, lane l: its two weight-row scales
};

struct TileScaleRegs {
  float xs, rw, b0, b1;
};

// Thread t: tile row t's scales (t < mrows <= 512 threads), and its lane's weight-row scales of
// the 64-column unit `unit` (a valid unit).
template <bool kGather, bool kSwiglu>
__device__ __forceinline__ TileScaleRegs load_tile_scales(const GemmArgs& g, const RowSrc& rs, int e,
                                                          int row0, int mrows, int unit) {
  const int tid = opaque_tid();
  const int rl = tid & 31;
  TileScaleRegs t{0.0f, 0.0f, 0.0f, 0.0f};
  if (tid < mrows) {
    t.xs = row_scale<kGather>(g, rs, row0 + tid);
    if (kSwiglu) t.rw = rs.weight(row0 + tid);
  }
  if (!kSwiglu) {
    t.b0 = g.b_scale[static_cast<int64_t>(e) * g.n + unit * 64 + rl];
    t.b1 = g.b_scale[static_cast<int64_t>(e) * g.n + unit * 64 + 32 + rl];
  } else {
    const int chan = unit * 32 + rl;
    t.b0 = g.b_scale[static_cast<int64_t>(e) * g.n + chan];
    t.b1 = g.b_scale[static_cast<int64_t>(e) * g.n + g.sw.inter + chan];
  }
  return t;
}

__device__ __forceinline__ void publish_tile_scales(TileTables& tt, const TileScaleRegs& t, int mrows) {
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  if (tid < mrows) {
    tt.xs[tid] = t.xs;
    tt.rw[tid] = t.rw;
  }
  tt.bs[wave][0][lane] = t.b0;
  tt.bs[wave][1][lane] = t.b1;
}

// Stores a wave's MT x (32 rows) x 64 columns of accumulators: rows [row0, row0 + mrows) of
// the output (mrows <= 32 * MT; table row trow0 + r holds row r's scales), 64-column unit `unit`
// of the output (SwiGLU: 32 channels).
// kCoherent: the stores go out device-coherent (sc1, written through the XCD's L2): GEMM2's
// partial rows, so that workgroups of other XCDs can read them in the same launch, and GEMM1's
// SwiGLU rows of the decode pipeline, which its GEMM2 items of the same XCD still read from L2
// but which no longer sit there dirty (c1 150.9 -> 148.9 us per layer; its y output rows written
// through as well made no difference, its act rows as 4-byte coherent stores +3 us).
// SwiGLU: y is stored in bf16 (the reference fused path's rounding of the activation before
// its quantization). kPmax (the decode pipeline's GEMM1): the row maxima of the rounded values
// are stored as well.
template <bool kSwiglu, int MT, bool kPmax = false, bool kCoherent = false>
__device__ __forceinline__ void store_tile(const GemmArgs& g, const v16f (&acc)[MT][2], int row0,
                                           int mrows, int unit, const TileTables& tt, int trow0) {
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int rl = lane & 31, hk = lane >> 5;
  const float b0 = tt.bs[wave][0][lane], b1 = tt.bs[wave][1][lane];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    // the 16 rows' table entries read at once (rows past mrows read entries never used)
    float xs[16], rw[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = mt * 32 + (v >> 2) * 8 + hk * 4 + (v & 3);
      xs[v] = tt.xs[trow0 + r];
      rw[v] = kSwiglu ? tt.rw[trow0 + r] : 0.0f;
    }
    float pm[16];  // kPmax: |y| of the lane's channel in each of its 16 rows
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      pm[v] = 0.0f;
      const int r = mt * 32 + (v >> 2) * 8 + hk * 4 + (v & 3);
      if (r >= mrows) continue;
      if (!kSwiglu) {
        uint16_t* crow = g.c + static_cast<int64_t>(row0 + r) * g.n + unit * 64 + rl;
        const uint16_t c0 = f32_to_bf16(acc[mt][0][v] * xs[v] * b0);
        const uint16_t c1 = f32_to_bf16(acc[mt][1][v] * xs[v] * b1);
        if constexpr (kCoherent) {
          __hip_atomic_store(crow, c0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(crow + 32, c1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          crow[0] = c0;
          crow[32] = c1;
        }
      } else {
        const float yv = swiglu_value(g, acc[mt][0][v], acc[mt][1][v], xs[v], b0, b1, rw[v]);
        const int64_t at = static_cast<int64_t>(row0 + r) * g.sw.inter + unit * 32 + rl;
        const uint16_t yb = f32_to_bf16(yv);
        if constexpr (kCoherent)
          __hip_atomic_store(g.sw.y + at, yb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          g.sw.y[at] = yb;
        if constexpr (kPmax) pm[v] = fabsf(bf16_to_f32(yb));
      }
    }
    if constexpr (kPmax && kSwiglu) {
      // the row maxima over the unit's 32 channels (the lanes of a half-wave); lane 16 + v of
      // each half writes row v of its half
#pragma unroll
      for (int v = 0; v < 16; ++v) pm[v] = half_wave_max_nonneg(pm[v]);
      float mv = pm[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) mv = (rl & 15) == v ? pm[v] : mv;
      const int v = rl & 15;
      const int r = mt * 32 + (v >> 2) * 8 + hk * 4 + (v & 3);
      if (rl >= 16 && r < mrows) g.row_pmax[static_cast<int64_t>(row0 + r) * (g.n / kStreamUnit) + unit] = mv;
    }
  }
}

// ------------------------------------------------------------------ STREAM engine
// The 8 waves of a STREAM tile step together: a bare s_barrier after every 64-k step (each wave
// has issued that step's ring refill before it, so the weight loads stay in flight). Left to
// themselves the waves drift apart -- the memory pipeline does not serve them evenly -- and a
// workgroup's first and last wave finished their streams 15-16 us apart at c1 (median), the
// last one 6-7 us after the median one, with fewer and fewer loads in flight at the end. In
// step, GEMM1 went from 109 to 97 us at c1 (a barrier every 4 steps: 103 us).
__device__ __forceinline__ void step_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup barrier for the LDS A chunks: this wave's LDS writes are complete, then s_barrier.
// It waits on no global load, so the weight loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16-byte piece p of LDS A row r sits at piece (p & ~7) | ((p ^ r) & 7): 8 lanes reading the
// same k of 8 consecutive rows hit 8 distinct 16-byte bank groups.
__device__ __forceinline__ int swizzle_piece(int p, int r) { return (p & ~7) | ((p ^ r) & 7); }

// One workgroup tile (expert e, 512-column block nb, rows [row0, row0 + mrows), mrows <= 32*MT)
// over the full K. kFast: K is a multiple of the chunk (2048/MT k), ring 4 steps deep (2 for
// four row tiles, whose 128 accumulators leave no room for more); else 128-k chunks and a
// one-step ring (small shapes).
//
// A chunk c+1 is loaded into registers (8 x 16 bytes per lane, whole 128-byte lines: lane l of
// load i covers LDS bytes gi*1024 + 16*l of the chunk buffer, gi = 8i + wave) right after the
// barrier that opens chunk c, and written to its LDS buffer at the end of chunk c, before the
// next barrier. Plain loads keep the memory counter in order, so every wait the compiler places
// for a weight step or for the staged chunk is exact; the chunk's loads are older than all
// weight loads of chunk c and cost no wait at all by then.
//
// kEarly: the weight ring's first steps go out first, then `before_a` runs (the decode
// pipeline's wait for the item's rows), then the item's scales and A rows are loaded.
// kAResident: before_a also leaves the item's whole A in the LDS chunk buffers (K of at most two
// chunks), so no A rows are loaded here.
struct NoHook {
  __device__ __forceinline__ void operator()() const {}
};
template <bool kGather, bool kSwiglu, int MT, bool kFast, bool kEarly = false, bool kAResident = false,
          bool kPmax = false, bool kCoherent = false, typename Hook = NoHook>
__device__ void stream_tile(const GemmArgs& g, const RowSrc& rs, int e, int row0, int mrows, int nb,
                            uint8_t* smem, TileTables& tt, const Hook& before_a = Hook{}) {
  static_assert(!kAResident || (kEarly && kFast), "a resident A is staged by the hook");
  // four row tiles: the accumulators take the registers of two ring steps
  constexpr int D = kFast ? (MT == 4 ? kStreamDepth / 2 : kStreamDepth) : 1;
  constexpr int kFullChunk = kAChunk / (32 * MT);  // k-bytes per chunk
  const int kc = kFast ? kFullChunk : 128;
  const int spc = kc / 64;  // steps per chunk
  const int nchunks = g.k / kc;
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int units = g.n / kStreamUnit;
  const int unit_raw = nb * kGemmWaves + wave;
  const bool active = unit_raw < units;  // a partial column block leaves waves without columns
  const int unit = active ? unit_raw : units - 1;

  const int chunk_bytes = 32 * MT * kc;
  const uint8_t* asrc[kALoads];
  auto a_sources = [&]() {  // (reads the row table: after before_a, which may fill it)
#pragma unroll
    for (int i = 0; i < kALoads; ++i) {
      const int pos = (i * kGemmWaves + wave) * 1024 + lane * 16;
      const int r = pos / kc;
      const int p = swizzle_piece((pos - r * kc) >> 4, r);
      asrc[i] = a_row_ptr<kGather>(g, rs, row0 + (r < mrows ? r : 0)) + p * 16;
    }
  };
  if constexpr (!kEarly) a_sources();
  int4 astage[kALoads];
  auto load_chunk = [&](int chunk) {
    if constexpr (kAResident) return;
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      if (kFast || (i * kGemmWaves + wave) * 1024 < chunk_bytes)
        astage[i] = ld16(asrc[i] + static_cast<int64_t>(chunk) * kc);
  };
  auto store_chunk = [&](int chunk) {
    if constexpr (kAResident) return;
    uint8_t* dst = smem + (chunk & 1) * kAChunk + wave * 1024 + lane * 16;
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      if (kFast || (i * kGemmWaves + wave) * 1024 < chunk_bytes)
        *reinterpret_cast<int4*>(dst + i * kGemmWaves * 1024) = astage[i];
  };
  // operand reads: lane l is row l%32 (+32 mt), k-bytes [64j + 32*(l/32), +32) of chunk step j
  const uint8_t* sbase = smem + (lane & 31) * kc;
  const int hk = lane >> 5;
  int pc[2][2];  // swizzled byte offset of piece 4v + 2hk + h within its 128-byte group
#pragma unroll
  for (int v = 0; v < 2; ++v)
#pragma unroll
    for (int h = 0; h < 2; ++h) pc[v][h] = (((4 * v + 2 * hk + h) ^ lane) & 7) << 4;

  const uint8_t* bp[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = weight_row<kSwiglu>(g, unit, kStreamUnit, ct * 32 + (lane & 31));
    bp[ct] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
             (n & 15) * 16 + hk * 512;
  }
  int4 br[D][2][2];  // [ring slot][column tile][16-byte half]
  auto issue = [&](int d, int s) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const uint8_t* p = bp[ct] + static_cast<int64_t>(s) * 1024;
      br[d][ct][0] = ld16_stream(p);
      br[d][ct][1] = ld16_stream(p + 256);
    }
  };
  v16f acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][ct][v] = 0.0f;
  // step j of chunk c (j & 1 is a compile-time constant in the unrolled loops below)
  auto compute = [&](int d, int c, int j) {
    const v8i b0 = make_v8i(br[d][0][0], br[d][0][1]);
    const v8i b1 = make_v8i(br[d][1][0], br[d][1][1]);
    const uint8_t* base = sbase + (c & 1) * kAChunk + (j >> 1) * 128;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint8_t* rb = base + mt * 32 * kc;
      const v8i a = make_v8i(*reinterpret_cast<const int4*>(rb + pc[j & 1][0]),
                             *reinterpret_cast<const int4*>(rb + pc[j & 1][1]));
      acc[mt][0] = mfma_fp8(a, b0, acc[mt][0]);
      acc[mt][1] = mfma_fp8(a, b1, acc[mt][1]);
    }
  };

  if constexpr (kEarly) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    before_a();
    if constexpr (!kAResident) a_sources();
  }
  // a resident A's hook also leaves the rows' scales in tt.xs
  const TileScaleRegs tsr = load_tile_scales<kGather, kSwiglu>(g, rs, e, row0, kAResident ? 0 : mrows, unit);
  load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kEarly) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  store_chunk(0);
  publish_tile_scales(tt, tsr, kAResident ? 0 : mrows);
  lds_barrier();
  for (int c = 0; c + 1 < nchunks; ++c) {
    load_chunk(c + 1);
    __builtin_amdgcn_sched_barrier(0);
    for (int j = 0; j < spc; j += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        compute(d, c, j + d);
        issue(d, c * spc + j + d + D);
        __builtin_amdgcn_sched_barrier(0);
        if (kFast) step_barrier();
      }
    }
    store_chunk(c + 1);  // its buffer was last read in chunk c - 1, before the last barrier
    lds_barrier();
  }
  {
    const int c = nchunks - 1;
    for (int j = 0; j + D < spc; j += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        compute(d, c, j + d);
        issue(d, c * spc + j + d + D);
        __builtin_amdgcn_sched_barrier(0);
        if (kFast) step_barrier();
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) compute(d, c, spc - D + d);
  }

  if (!active) return;
  store_tile<kSwiglu, MT, kPmax, kCoherent>(g, acc, row0, mrows, unit, tt, 0);
}

// ------------------------------------------------------------------ TILE engine
// One 256 x 256 output tile (expert e, 256-column block nb, rows [row0, row0 + mrows)), K in
// BK = 128 stages through double-buffered LDS: the next stage's global loads go out into
// registers before the MFMAs of the current one and are written to the other LDS stage after
// them (one barrier per stage). A stage holds A as 256 rows of 128 bytes, 16-byte piece p of
// row r at piece p ^ (r % 8) (loaded as whole lines: 8 lanes per row), then B in Marlin's own
// blocks (16 row-tiles x 8 k-blocks x 256 bytes: each row-tile's stage is 2 KB contiguous in
// the weight, copied as is). A 32x32x64 operand is two 16-byte LDS reads per lane; 16 lanes
// read 256 contiguous bytes of B, and 8 lanes read 8 distinct 16-byte bank groups of A.
template <bool kGather, bool kSwiglu>
__device__ void tile_tile(const GemmArgs& g, const RowSrc& rs, int e, int row0, int mrows, int nb,
                          uint8_t* smem, TileTables& tt) {
  constexpr int BK = kTileBK;
  constexpr int TM = kTileBM / kTileWM / 32, TN = kTileBN / kTileWN / 32;  // 4 x 2
  constexpr int kALoads = kTileBM * BK / 16 / kGemmThreads;  // 4
  constexpr int kBLoads = kTileBN * BK / 16 / kGemmThreads;  // 4
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / kTileWN, wn = wave % kTileWN;
  const int k_steps = g.k / BK;
  const int units = g.n / kStreamUnit;            // 64-column units of the output
  const int unit = nb * kTileWN + wn;             // this wave's unit
  const int row_tiles = g.n / 16;                 // weight row-tiles of the expert

  // A: load i covers rows i*64 + tid/8, piece tid % 8 (whole 128-byte row lines); stored at
  // piece p ^ ((r / 2) % 8), so 16 consecutive rows at one k hit 16 distinct bank groups
  const uint8_t* a_src[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int r = i * (kGemmThreads / 8) + (tid >> 3);
    a_src[i] = a_row_ptr<kGather>(g, rs, row0 + (r < mrows ? r : 0)) + (tid & 7) * 16;
  }
  const int a_key = (tid >> 4) & 7;  // (r / 2) % 8 of every A row this thread stores
  const int a_dst0 = (tid >> 3) * BK + (((tid & 7) ^ a_key) << 4);  // + i * 64 * BK
  // B: load i covers byte q = (i*512 + tid)*16 of the stage's 16 row-tiles x 2 KB
  const uint8_t* b_src[kBLoads];
#pragma unroll
  for (int i = 0; i < kBLoads; ++i) {
    const int q = (i * kGemmThreads + tid) * 16;
    const int rt = q >> 11;  // 2 KB per row-tile per stage
    int n = weight_row<kSwiglu>(g, nb, kTileBN, rt * 16);
    if ((n >> 4) >= row_tiles) n = 0;  // a partial column block: any valid row-tile
    b_src[i] = g.b + (static_cast<int64_t>(e) * row_tiles + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
               (q & 2047);
  }
  int4 ra[kALoads], rb[kBLoads];
  auto load_stage = [&](int kt) {
#pragma unroll
    for (int i = 0; i < kALoads; ++i) ra[i] = ld16(a_src[i] + kt * BK);
#pragma unroll
    for (int i = 0; i < kBLoads; ++i) rb[i] = ld16(b_src[i] + static_cast<int64_t>(kt) * BK * 16);
  };
  auto store_stage = [&](int buf) {
    uint8_t* sa = smem + buf * kTileStage;
    uint8_t* sb = sa + kTileBM * BK;
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      *reinterpret_cast<int4*>(sa + a_dst0 + i * (kGemmThreads / 8) * BK) = ra[i];
#pragma unroll
    for (int i = 0; i < kBLoads; ++i) *reinterpret_cast<int4*>(sb + (i * kGemmThreads + tid) * 16) = rb[i];
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // B column of the wave's column tile tn: without SwiGLU wn*64 + tn*32; with SwiGLU the
  // gate columns (tn = 0) at wn*32 and the matching up columns (tn = 1) at 128 + wn*32.
  auto b_col = [&](int tn) { return kSwiglu ? tn * (kTileBN / 2) + wn * 32 : wn * 64 + tn * 32; };
  const int hk = lane >> 5;
  const int rkey = ((lane & 31) >> 1) & 7;  // (r / 2) % 8 of this lane's A rows
  // Operands are read one MFMA group ahead (double-buffered registers), so the LDS latency of
  // the next A (or the next k-step's B) overlaps the MFMAs of the current one.
  auto read_b = [&](const uint8_t* sb, int ks, v8i (&bv)[TN]) {
    const int p0 = ks * 4 + hk * 2;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int c = b_col(tn) + (lane & 31);
      const uint8_t* bc = sb + (c >> 4) * (BK * 16) + p0 * 256 + (c & 15) * 16;
      bv[tn] = make_v8i(*reinterpret_cast<const int4*>(bc), *reinterpret_cast<const int4*>(bc + 256));
    }
  };
  auto read_a = [&](const uint8_t* sa, int ks, int tm) {
    const int p0 = ks * 4 + hk * 2;
    const uint8_t* ar = sa + (wm * (TM * 32) + tm * 32 + (lane & 31)) * BK;
    return make_v8i(*reinterpret_cast<const int4*>(ar + ((p0 ^ rkey) << 4)),
                    *reinterpret_cast<const int4*>(ar + (((p0 + 1) ^ rkey) << 4)));
  };
  auto compute_stage = [&](int buf) {
    const uint8_t* sa = smem + buf * kTileStage;
    const uint8_t* sb = sa + kTileBM * BK;
    v8i bv[2][TN];
    read_b(sb, 0, bv[0]);
    v8i a_cur = read_a(sa, 0, 0);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        v8i a_next;
        if (tm + 1 < TM) a_next = read_a(sa, ks, tm + 1);
        else if (ks + 1 < BK / 64) {
          read_b(sb, ks + 1, bv[(ks + 1) & 1]);
          a_next = read_a(sa, ks + 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs below
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = mfma_fp8(a_cur, bv[ks & 1][tn], acc[tm][tn]);
        __builtin_amdgcn_sched_barrier(0);
        a_cur = a_next;
      }
    }
  };

  // a partial column block leaves waves without columns: their scales come from any valid unit
  const TileScaleRegs tsr =
      load_tile_scales<kGather, kSwiglu>(g, rs, e, row0, mrows, unit < units ? unit : units - 1);
  load_stage(0);
  store_stage(0);
  publish_tile_scales(tt, tsr, mrows);
  __syncthreads();
  for (int kt = 0; kt < k_steps; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < k_steps) load_stage(kt + 1);
    compute_stage(cur);
    if (kt + 1 < k_steps) store_stage(cur ^ 1);
    __syncthreads();
  }
  if (unit >= units) return;
  static_assert(TN == 2 && TM == 4, "a wave's tile is 128 rows x 64 columns");
  const int wrow = row0 + wm * (TM * 32);
  const int wrows = mrows - wm * (TM * 32);
  store_tile<kSwiglu, 2>(g, *reinterpret_cast<const v16f(*)[2][2]>(&acc[0]), wrow, wrows, unit, tt,
                         wm * (TM * 32));
  store_tile<kSwiglu, 2>(g, *reinterpret_cast<const v16f(*)[2][2]>(&acc[2]), wrow + 64, wrows - 64,
                         unit, tt, wm * (TM * 32) + 64);
}

// ------------------------------------------------------------------ WIDE engine
// The TILE engine's 256 x 256 tile for a 4-wave workgroup (one wave per SIMD: 512 registers a
// lane, the 256 accumulators in AGPRs), used when every expert has many rows. Wave w owns the
// 64-column unit nb*4 + w over all 256 rows (8 x 2 MFMA tiles), so each weight column is read
// by one wave only: B goes straight from global memory into MFMA operand registers (Marlin
// gives each lane 16 contiguous k-bytes of a weight row), four 64-k steps ahead in a register
// ring, and never touches LDS. A goes through LDS in BK = 128 stages: 256 rows of 128 bytes,
// 16-byte piece p of row r at piece p ^ ((r / 2) % 8) (16 consecutive rows at one k hit 16
// distinct 16-byte bank groups), three stages deep, so the first A operand of a stage is read
// before the barrier that ends the previous one and the MFMA pipe does not drain there. A
// stage's A is loaded one stage before its LDS write, spread one load or one LDS write per MFMA
// group. Tiles are independent (prologue, stages, epilogue): a software pipeline across the
// tiles of a workgroup needed the next tile's offsets live through the stage loop and the
// compiler spilled (measured slower).
//
// Two shapes (BM = rows of a full tile): BM = 256 with one workgroup per CU (512 registers a
// lane), and BM = 128 with two workgroups per CU (256 registers a lane, 128 AGPR accumulators):
// then each SIMD runs two waves of different tiles, and one tile's prologue and epilogue overlap
// the other's MFMAs. The B ring and the A operand look-ahead are shallower at BM = 128 (the
// other wave covers the latency).
constexpr int kWideThreads = 256, kWideWaves = 4;
constexpr int kWideBK = 128;
constexpr int kWideBufs = 3;
constexpr int kWideMinRowsPerExpert = kTileBM;  // average routed rows that select it

template <int BM>
struct WideShape {
  static_assert(BM == 256 || BM == 128, "full tile of 256 or 128 rows");
  static constexpr int kStage = BM * kWideBK;  // bytes of one A stage
  // after the A ring, the tile's tables: BM row scales, the 256 weight-row scales (f32), then
  // (GEMM2) BM row addresses (u64)
  static constexpr int kTables = kWideBufs * kStage;
  static constexpr int kColScales = BM * 4;
  static constexpr int kAddrs = kColScales + kWideWaves * kStreamUnit * 4;
  static constexpr int kSmemBytes = kTables + kAddrs + BM * 8;
  static constexpr int kRing = BM == 256 ? 4 : 2;  // 64-k steps of B in registers
  static constexpr int kWavesPerSimd = BM == 256 ? 1 : 2;
  static constexpr int kFullTM = BM / 32;
  // the epilogue stages each wave's 64 output rows (8 KB) in the A ring's first bytes
  static_assert(kWideWaves * 8192 <= kTables, "epilogue staging fits the A ring");
};

// Epilogue of a WIDE tile. The MFMAs run transposed (weights as the first operand), so lane
// l holds token row tm*32 + l%32 and, per 32-column tile tn, the columns 8*(v/4) + 4*(l/32) +
// v%4: four runs of 4 consecutive columns. The row scale is then one value per lane and row
// tile, the column scales four 16-byte LDS reads per column tile (both from the tile's scale
// table), and every 4 results become one 8-byte bf16 write into the wave's 8 KB slice of a
// free 32 KB A buffer (64 rows x 128 bytes, 16-byte piece p of row r at p ^ ((r / 2) % 8):
// conflict-free both ways); each pass of 64 rows then leaves as whole 16-byte pieces, 8 rows
// per store instruction.
// GEMM2 writes the bf16 partials (-0 as +0) to the row addresses of the tile's table: its part
// row, or for a row whose token has no other routed slot its y row (row_dest).
template <int BM, int TM>
__device__ __forceinline__ void store_wide(const GemmArgs& g, const v16f (&acc)[TM][2], int row0,
                                           int mrows, int unit, uint8_t* stage,
                                           const uint8_t* table) {
  using W = WideShape<BM>;
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1);
  const int rl = lane & 31, hk = lane >> 5;
  const float* s_xs = reinterpret_cast<const float*>(table);
  const float* s_bs = reinterpret_cast<const float*>(table + W::kColScales) + (tid / kWave) * kStreamUnit;
  const uint64_t* s_addr = reinterpret_cast<const uint64_t*>(table + W::kAddrs);
  float4 bs[2][4];
#pragma unroll
  for (int tn = 0; tn < 2; ++tn)
#pragma unroll
    for (int q = 0; q < 4; ++q) bs[tn][q] = *reinterpret_cast<const float4*>(s_bs + tn * 32 + q * 8 + hk * 4);
  uint8_t* wlds = stage + (tid / kWave) * 8192;
  const int piece = lane & 7;
  const int col = unit * 64 + piece * 8;
#pragma unroll
  for (int pass = 0; pass < (TM + 1) / 2; ++pass) {
#pragma unroll
    for (int t2 = 0; t2 < (TM > 1 ? 2 : 1); ++t2) {  // TM = 1: one row tile, rows 32-63 unused
      const int tm = pass * 2 + t2;
      const float xs = s_xs[tm * 32 + rl];
      const int r = t2 * 32 + rl;  // row within the pass
      const int rkey = (r >> 1) & 7;
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 ws = bs[tn][q];
          // the scale product as fma(., ., +0), the same rounding, but a zero is +0 (the
          // combine's sum from +0 writes +0 too, so a y row written here matches it bitwise)
          auto scaled = [&](float a, float w) { return __builtin_fmaf(a * xs, w, 0.0f); };
          const uint32_t lo = pack_bf16x2(scaled(acc[tm][tn][4 * q], ws.x), scaled(acc[tm][tn][4 * q + 1], ws.y));
          const uint32_t hi = pack_bf16x2(scaled(acc[tm][tn][4 * q + 2], ws.z), scaled(acc[tm][tn][4 * q + 3], ws.w));
          // columns tn*32 + 8q + 4hk .. +4 -> bytes 64tn + 16q + 8hk: piece 4tn + q, half hk
          const int pc = (4 * tn + q) ^ rkey;
          *reinterpret_cast<uint2*>(wlds + r * 128 + pc * 16 + hk * 8) = make_uint2(lo, hi);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's LDS writes before its reads
    int4 val[8];
    uint64_t base[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = i * 8 + (lane >> 3);
      val[i] = *reinterpret_cast<const int4*>(wlds + rr * 128 + ((piece ^ ((rr >> 1) & 7)) << 4));
      base[i] = s_addr[pass * 64 + rr];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int grow = pass * 64 + i * 8 + (lane >> 3);
      // the row's address from the table (its part row or its token's y row); a global (not
      // flat) store: a flat one would also hold up the LDS counter. Nontemporal: the rows are
      // read once, by the combine (c3 -25 us)
      const i32x4 v = {val[i].x, val[i].y, val[i].z, val[i].w};
      if (grow < mrows)
        __builtin_nontemporal_store(v, (__attribute__((address_space(1))) i32x4*)(base[i] + col * 2));
    }
    // the next pass's LDS writes follow these reads in the wave's own (in-order) LDS queue
  }
}

// Epilogue of a WIDE GEMM1 tile with the SwiGLU: the wave's unit holds the gate channels
// unit*32 + c (column tile 0) and the up channels of the same c (column tile 1), so lane l has,
// for token row tm*32 + l%32, four runs of 4 channels 8q + 4*(l/32) .. + 4 of both. Per channel:
// g = bf16(acc_g * x_scale * w_scale_g) and u = bf16(acc_u * x_scale * w_scale_u) (the staged
// K1 output h, rounded like its stores), then y = SwiGLU(g, u) x route weight (the K2 formula,
// with the activation clamp when kClamp) and y rounded to bf16: bf16 y [rows, I] for the
// requant, half of h's bytes. Each 4-channel run is one 8-byte write into the wave's 4 KB LDS
// slice (64 rows x 64 bytes, 16-byte piece p of row r at p ^ ((r / 4) % 4)); a pass of 64 rows
// leaves as 16-byte pieces, 16 rows per store instruction.
template <bool kClamp, int BM, int TM>
__device__ __forceinline__ void store_wide_swiglu(const GemmArgs& g, const v16f (&acc)[TM][2], int row0,
                                                  int mrows, int unit, uint8_t* stage,
                                                  const uint8_t* table) {
  using W = WideShape<BM>;
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1);
  const int rl = lane & 31, hk = lane >> 5;
  const float* s_xs = reinterpret_cast<const float*>(table);
  const float* s_rw = reinterpret_cast<const float*>(table + W::kAddrs);  // route weights
  const float* s_bs = reinterpret_cast<const float*>(table + W::kColScales) + (tid / kWave) * kStreamUnit;
  float4 bs[2][4];
#pragma unroll
  for (int tn = 0; tn < 2; ++tn)
#pragma unroll
    for (int q = 0; q < 4; ++q) bs[tn][q] = *reinterpret_cast<const float4*>(s_bs + tn * 32 + q * 8 + hk * 4);
  uint8_t* wlds = stage + (tid / kWave) * 4096;
  const int64_t ld = g.sw.inter;
  uint16_t* out = g.sw.y + static_cast<int64_t>(row0) * ld + unit * 32 + (lane & 3) * 8;
  const float cv = g.sw.clamp;
#pragma unroll
  for (int pass = 0; pass < (TM + 1) / 2; ++pass) {
#pragma unroll
    for (int t2 = 0; t2 < (TM > 1 ? 2 : 1); ++t2) {  // TM = 1: one row tile, rows 32-63 unused
      const int tm = pass * 2 + t2;
      const float xs = s_xs[tm * 32 + rl];
      const float rw = s_rw[tm * 32 + rl];
      const int r = t2 * 32 + rl;  // row within the pass
      const int rkey = (r >> 2) & 3;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 wg = bs[0][q], wu = bs[1][q];
        const v16f& ag = acc[tm][0];
        const v16f& au = acc[tm][1];
        // gate and up of a channel rounded to bf16 together (one conversion for the pair)
        auto y_of = [&](float a_g, float a_u, float w_g, float w_u) {
          const uint32_t h = pack_bf16x2(a_g * xs * w_g, a_u * xs * w_u);
          return swiglu_weighted_c<kClamp>(__uint_as_float(h << 16), __uint_as_float(h & 0xffff0000u), rw, cv);
        };
        const float y0 = y_of(ag[4 * q], au[4 * q], wg.x, wu.x);
        const float y1 = y_of(ag[4 * q + 1], au[4 * q + 1], wg.y, wu.y);
        const float y2 = y_of(ag[4 * q + 2], au[4 * q + 2], wg.z, wu.z);
        const float y3 = y_of(ag[4 * q + 3], au[4 * q + 3], wg.w, wu.w);
        // channels 8q + 4hk .. +4 -> bytes 16q + 8hk of the row: piece q, half hk
        *reinterpret_cast<uint2*>(wlds + r * 64 + ((q ^ rkey) << 4) + hk * 8) =
            make_uint2(pack_bf16x2(y0, y1), pack_bf16x2(y2, y3));
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's LDS writes before its reads
    int4 val[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = i * 16 + (lane >> 2);
      val[i] = *reinterpret_cast<const int4*>(wlds + rr * 64 + (((lane & 3) ^ ((rr >> 2) & 3)) << 4));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int grow = pass * 64 + i * 16 + (lane >> 2);
      if (grow < mrows) *reinterpret_cast<int4*>(out + grow * ld) = val[i];
    }
    // the next pass's LDS writes follow these reads in the wave's own (in-order) LDS queue
  }
}

// TM row tiles of 32: BM/32 for a full tile; fewer (4, 2 or 1) for an expert's last tile of
// at most 128, 64 or 32 rows (a fraction of the MFMAs and A traffic for the row remainder).
template <bool kGather, bool kSwiglu, int BM, int TM, typename Hook = NoHook>
__device__ void wide_tile(const GemmArgs& g, const RowSrc& rs, int e, int row0, int mrows, int nb,
                          uint8_t* smem, const Hook& before_epilogue = Hook{}) {
  using W = WideShape<BM>;
  constexpr int kWideStage = W::kStage;
  constexpr int kWideTables = W::kTables;
  constexpr int kWideRing = W::kRing;
  static_assert(TM <= W::kFullTM, "a tile of at most BM rows");
  constexpr int TN = kStreamUnit / 32;                        // 2
  constexpr int kALoads = TM * 32 * kWideBK / 16 / kWideThreads;  // TM
  constexpr int kRowsPerLoad = kWideThreads / (kWideBK / 16);     // 32
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int stages = g.k / kWideBK;
  const int steps = stages * (kWideBK / 64);
  const int units = g.n / kStreamUnit;
  const int unit_raw = nb * kWideWaves + wave;
  const bool active = unit_raw < units;
  const int unit = active ? unit_raw : units - 1;  // a partial column block: any valid columns
  const int hk = lane >> 5;

  // A: load i covers row i*32 + tid/8, piece tid % 8 (rows past mrows read row 0). GEMM1
  // (gather): the row scales for the epilogue's table are loaded by the same threads, from the
  // same tokens (the eight threads of a row read one word and write one LDS entry with the same
  // value), all the tokens first and then all the scales, with no branch between them, ahead of
  // the stages' loads, so that every wait the compiler places in the prologue is exact (a scale
  // chain of its own, token -> scale, had been sunk behind all the stage loads and made the
  // prologue wait for every one of them). GEMM2 loads one row scale a thread (no chain).
  const uint8_t* a_src[kALoads];
  float a_rs[kALoads];
  int64_t a_row[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int r = i * kRowsPerLoad + (tid >> 3);
    const int row = row0 + (r < mrows ? r : 0);
    a_row[i] = kGather ? static_cast<int64_t>(rs.token(row)) : row;
  }
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    a_src[i] = g.a + a_row[i] * g.lda + (tid & 7) * 16;
    a_rs[i] = kGather ? g.a_scale[a_row[i]] : 0.0f;
  }
  const float pre_xs = kGather ? 0.0f : g.a_scale[row0 + min(tid, mrows - 1)];
  const int a_dst0 = (tid >> 3) * kWideBK + (((tid & 7) ^ ((tid >> 4) & 7)) << 4);
  // two register sets: a stage's A is loaded one stage before it is written to LDS, which is
  // one stage before it is read
  int4 ra[2][kALoads];
  auto load_a = [&](int set, int i, int kt) { ra[set][i] = ld16(a_src[i] + kt * kWideBK); };
  auto store_a = [&](int set, int i, int kt) {
    *reinterpret_cast<int4*>(smem + (kt % kWideBufs) * kWideStage + a_dst0 + i * kRowsPerLoad * kWideBK) =
        ra[set][i];
  };
  // B: column tile tn of the wave's unit; 64-k step s of the lane's column at + s*1024 (+256)
  const uint8_t* bp[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int n = weight_row<kSwiglu>(g, unit, kStreamUnit, tn * 32 + (lane & 31));
    bp[tn] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
             (n & 15) * 16 + hk * 512;
  }
  int4 br[kWideRing][TN][2];
  auto load_b = [&](int slot, int s) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const uint8_t* q = bp[tn] + static_cast<int64_t>(s) * 1024;
      br[slot][tn][0] = ld16(q);
      br[slot][tn][1] = ld16(q + 256);
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int rkey = ((lane & 31) >> 1) & 7;
  auto read_a = [&](int kt, int ks, int tm) {
    const int p0 = ks * 4 + hk * 2;
    const uint8_t* ar = smem + (kt % kWideBufs) * kWideStage + (tm * 32 + (lane & 31)) * kWideBK;
    return make_v8i(*reinterpret_cast<const int4*>(ar + ((p0 ^ rkey) << 4)),
                    *reinterpret_cast<const int4*>(ar + (((p0 + 1) ^ rkey) << 4)));
  };
  // A stage = 16 MFMA groups (2 steps x 8 row tiles, 2 MFMAs each). The A operand of group
  // g + 3 is read while group g's MFMAs run (ring of 4 operands; the last groups read the next
  // stage's first operands, whose buffer is complete since the previous barrier), which
  // covers the LDS latency with one wave per SIMD. Order pinned by sched_barrier.
  constexpr int kGroups = (kWideBK / 64) * TM;
  // one wave a SIMD: read 3 groups ahead; two (BM = 128): 1; TM = 1 has two groups a stage
  constexpr int kAhead = W::kWavesPerSimd == 1 ? (kGroups >= 4 ? 3 : kGroups - 1) : 1;
  static_assert(kGroups % (kAhead + 1) == 0, "operand ring index must repeat per stage");
  v8i abuf[kAhead + 1];
  auto read_group = [&](int kt, int gi) {
    const int g2 = gi % kGroups;
    return read_a(kt + gi / kGroups, g2 / TM, g2 % TM);
  };
  const int last_step = steps - 1;
  const int last_stage = stages - 1;
  // stage kt: 16 groups; groups 0-7 each load one piece of stage kt + 3's A into register set
  // `lset`, groups 8-15 each write one piece of stage kt + 2's A (set `wset`, loaded during
  // the previous stage) into its LDS buffer, each step's last group refills its B ring slot
  // with the step 4 ahead; then the barrier. Spread out, these loads and LDS writes issue in
  // the gaps between MFMAs instead of stalling the MFMA pipe in bursts.
  auto stage = [&](int kt, int slot0, int wset, int lset) {
    const int kt_load = min(kt + 3, last_stage);
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
      const int ks = gi / TM, tm = gi % TM;
      abuf[(gi + kAhead) % (kAhead + 1)] = read_group(kt, gi + kAhead);
      if (gi < kALoads) load_a(lset, gi, kt_load);
      else store_a(wset, gi - kALoads, kt + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        acc[tm][tn] = mfma_fp8(make_v8i(br[slot0 + ks][tn][0], br[slot0 + ks][tn][1]),
                               abuf[gi % (kAhead + 1)], acc[tm][tn]);  // transposed tile
      __builtin_amdgcn_sched_barrier(0);
      if (tm == TM - 1) {
        load_b(slot0 + ks, min(kt * (kWideBK / 64) + ks + kWideRing, last_step));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    lds_barrier();
  };
  static_assert(kGroups == 2 * kALoads, "one A load and one A write per group");

  // prologue: the epilogue's scales (the row scales loaded with the row tokens above; thread
  // t: the weight-row scale of its wave's column lane), A stages 0 and 1 into LDS, stage 2 into
  // register set 0, B steps 0..3, the first operands; the loads of stages 0, 1 and 2 go out
  // together (stage 0 through registers of the prologue's own), so that stage 2 is in before
  // the first stage needs it.
  // GEMM2: row tid's output address (its part row, or its token's y row when the token has no
  // other routed slot and direct rows are on); the switch and the row table load side by side.
  // Rows past mrows take the last row's (never stored).
  int pre_dest = -1, pre_on = 0;
  if (!kSwiglu && g.y_direct != nullptr) {
    pre_on = *g.direct_flag;
    pre_dest = g.row_dest[row0 + min(tid, mrows - 1)];
  }
  // GEMM1: row tid's route weight (the SwiGLU epilogue's)
  const float pre_rw = kSwiglu ? g.sw.row_weight[row0 + min(tid, mrows - 1)] : 0.0f;
  const float pre_bs = g.b_scale[static_cast<int64_t>(e) * g.n + weight_row<kSwiglu>(g, unit, kStreamUnit, lane)];
  int4 ra0[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) ra0[i] = ld16(a_src[i]);
#pragma unroll
  for (int i = 0; i < kALoads; ++i) load_a(1, i, min(1, last_stage));
#pragma unroll
  for (int i = 0; i < kALoads; ++i) load_a(0, i, min(2, last_stage));
#pragma unroll
  for (int sl = 0; sl < kWideRing; ++sl) load_b(sl, min(sl, last_step));
#pragma unroll
  for (int i = 0; i < kALoads; ++i)
    *reinterpret_cast<int4*>(smem + a_dst0 + i * kRowsPerLoad * kWideBK) = ra0[i];  // stage 0, buffer 0
#pragma unroll
  for (int i = 0; i < kALoads; ++i) store_a(1, i, 1);
  if constexpr (kGather) {
#pragma unroll
    for (int i = 0; i < kALoads; ++i) reinterpret_cast<float*>(smem + kWideTables)[i * kRowsPerLoad + (tid >> 3)] = a_rs[i];
  } else if (tid < BM) {
    reinterpret_cast<float*>(smem + kWideTables)[tid] = pre_xs;
  }
  reinterpret_cast<float*>(smem + kWideTables + W::kColScales)[tid] = pre_bs;
  if (kSwiglu && (BM == kWideThreads || tid < BM)) reinterpret_cast<float*>(smem + kWideTables + W::kAddrs)[tid] = pre_rw;
  if (!kSwiglu && (BM == kWideThreads || tid < BM)) {
    const int prow = row0 + min(tid, mrows - 1);
    reinterpret_cast<uint64_t*>(smem + kWideTables + W::kAddrs)[tid] =
        pre_on != 0 && pre_dest >= 0 ? reinterpret_cast<uint64_t>(g.y_direct + static_cast<int64_t>(pre_dest) * g.n)
                                     : reinterpret_cast<uint64_t>(g.c + static_cast<int64_t>(prow) * g.n);
  }
  lds_barrier();
#pragma unroll
  for (int gi = 0; gi < kAhead; ++gi) abuf[gi] = read_group(0, gi);
  // two stages per iteration, so that the ring slots are compile-time indices; every load is
  // issued unconditionally (past the end it reloads the last step or stage), which keeps the
  // compiler's load counting exact
  for (int kt = 0; kt < stages; kt += 2) {  // stages is even (k % 256 == 0)
    stage(kt, 0, 0, 1);
    stage(kt + 1, kWideRing == 4 ? 2 : 0, 1, 0);  // a ring of 2 refills the same two slots
  }
  // every wave has passed its last LDS read of A (the barrier that ended the last stage)
  before_epilogue();
  if (!active) return;
  if constexpr (kSwiglu) {
    if (g.sw.has_clamp) store_wide_swiglu<true, BM, TM>(g, acc, row0, mrows, unit, smem, smem + kWideTables);
    else store_wide_swiglu<false, BM, TM>(g, acc, row0, mrows, unit, smem, smem + kWideTables);
  } else {
    store_wide<BM, TM>(g, acc, row0, mrows, unit, smem, smem + kWideTables);
  }
}

// ------------------------------------------------------------------ in-kernel routing
// For small task counts GEMM1 routes the tokens itself instead of a separate routing kernel:
// every workgroup counts all tasks with its 8 waves (LDS atomics into per-wave counts; integer
// sums, so order-free and deterministic), keeps each task's expert in an LDS byte table, turns
// the counts into per-wave bases and expert offsets, and plans the items. For an item it then
// ranks only its own expert's tasks (one ballot per 64 tasks from the LDS table, ascending
// task order as in the routing kernels) into an LDS row table of tokens and route weights.
// The workgroup holding column block 0 of a row range writes that range's routing outputs
// (row_token, row_weight, m_indices, output_index) for the later stages; workgroup 0 writes
// counts, offsets, meta, stats and the -1 of the invalid tasks.
constexpr int kFusedPasses = 16;  // 64-task passes per wave
constexpr int kFusedMaxTasks = kGemmWaves * kFusedPasses * kWave;
constexpr int kFusedMaxExperts = 255;  // expert ids in a byte, 255 = invalid task
constexpr int kFusedBatch = 16;        // passes whose loads are in flight together
constexpr int kRowTable = kTileBM;  // LDS row table: one TILE's 256 rows

__device__ __forceinline__ int fused_per_wave(int ntasks) {
  return (ntasks + kGemmWaves * kWave - 1) / (kGemmWaves * kWave) * kWave;
}

// Per-wave counts of all tasks into s_wcnt[wave][e] and each task's expert into s_ev;
// workgroup 0 also marks the invalid tasks.
__device__ void fused_count(const RouteArgs& a, int ntasks, int (*s_wcnt)[kMaxGemmExperts],
                            uint8_t* s_ev, float* s_task_w, bool publisher) {
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int per = fused_per_wave(ntasks);
  const int begin = wave * per;
  const int end = min(begin + per, ntasks);
  for (int b = begin; b < end; b += kFusedBatch * kWave) {
    int ev[kFusedBatch];
    float wv[kFusedBatch];
    wave_load<kFusedBatch>(a, b, end, ev, wv);
#pragma unroll
    for (int p = 0; p < kFusedBatch; ++p) {
      const int task = b + p * kWave + lane;
      if (task < end) {
        s_ev[task] = ev[p] < 0 ? 255 : static_cast<uint8_t>(ev[p]);
        s_task_w[task] = wv[p];
        if (ev[p] >= 0) atomicAdd(&s_wcnt[wave][ev[p]], 1);
        else if (publisher) a.output_index[task] = -1;
      }
    }
  }
}

// Rows [r_lo, r_lo + kRowTable) of expert e (cnt rows): tokens and route weights into the LDS
// row table; rows in [w_lo0, w_hi0) or [w_lo1, w_hi1) are this workgroup's to write out.
// Ends with the table complete (workgroup barrier).
__device__ void fused_rows(const RouteArgs& a, int ntasks, int e, int cnt, int off_e,
                           const int (*s_wcnt)[kMaxGemmExperts], const uint8_t* s_ev,
                           const float* s_task_w, int r_lo, int w_lo0, int w_hi0, int w_lo1,
                           int w_hi1, int* s_task, int* s_tok, float* s_rw) {
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int per = fused_per_wave(ntasks);
  const int begin = wave * per;
  const int end = min(begin + per, ntasks);
  int run = s_wcnt[wave][e];  // rank of the wave's first task of expert e
  for (int b = begin; b < end; b += kWave) {
    const int task = b + lane;
    const int ev = task < end ? s_ev[task] : 255;
    const uint64_t m = __ballot(ev == e);
    if (ev == e) {
      const int rank = run + __popcll(m & lanes_below());
      if (rank >= r_lo && rank < r_lo + kRowTable) {
        s_task[rank - r_lo] = task;
        s_tok[rank - r_lo] = task / a.topk;
      }
    }
    run += __popcll(m);
  }
  __syncthreads();
  const int n = min(kRowTable, cnt - r_lo);
  for (int t = opaque_tid(); t < n; t += kGemmThreads) {  // recomputed, not kept live across items
    const int task = s_task[t];
    const float w = s_task_w != nullptr ? s_task_w[task] : a.topk_w[task];
    s_rw[t] = w;
    const int rank = r_lo + t;
    if ((rank >= w_lo0 && rank < w_hi0) || (rank >= w_lo1 && rank < w_hi1)) {
      const int64_t row = static_cast<int64_t>(off_e) + rank;
      const int out = row < a.row_cap ? static_cast<int>(row) : -1;
      // device-coherent: the decode pipeline's combine reads it from other XCDs
      __hip_atomic_store(&a.output_index[task], out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (out >= 0) {
        a.row_token[out] = s_tok[t];
        if (a.row_weight != nullptr) a.row_weight[out] = w;
        if (a.m_indices != nullptr) a.m_indices[out] = e;
      }
    }
  }
  __syncthreads();
}

// Wave 0: the per-wave counts s_wcnt[w][e] -> per-wave bases (the wave's first rank of each
// expert), the expert totals s_count[e] and their exclusive scan s_off[0..E] (expert offsets).
// The LDS traffic of one wave stays in order, so a plan by the same wave can follow at once.
__device__ void fused_scan(int E, int (*s_wcnt)[kMaxGemmExperts], int* s_count, int* s_off) {
  const int lane = lane_id();
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    int run = 0;
    if (e < E) {
      for (int w = 0; w < kGemmWaves; ++w) {
        const int c = s_wcnt[w][e];
        s_wcnt[w][e] = run;
        run += c;
      }
      s_count[e] = run;
    }
    const int inc = wave_inclusive_sum(run);
    if (e < E) s_off[e] = carry + inc - run;
    carry += __shfl(inc, kWave - 1, kWave);
  }
  if (lane == 0) s_off[E] = carry;
}

// ------------------------------------------------------------------ persistent dispatcher
__device__ __forceinline__ int stream_blocks(const GemmArgs& g) {
  return (g.n / kStreamUnit + kGemmWaves - 1) / kGemmWaves;
}

// Wave 0 fills s_prefix[0..E] with the exclusive prefix of the workgroup work items of the
// experts and s_tile[e] with the expert's engine (1 = TILE), from the routed rows s_count[e].
// A STREAM item is one (128-row chunk, 512-column block), an expert's chunks of one column
// block next to each other; a TILE item is one 256 x 256 tile (tile_coords' order).
__device__ void plan_items(const GemmArgs& g, int* s_prefix, int* s_tile, const int* s_count,
                           bool all_tile = false, int tile_rows = kTileBM) {
  const int E = g.num_experts;
  const int lane = lane_id();
  const int stream_nb = stream_blocks(g);
  const int tile_nb = (g.n + kTileBN - 1) / kTileBN;
  if (threadIdx.x < kWave) {
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int e = e0 + lane;
      int items = 0;
      if (e < E) {
        const int cnt = s_count[e];
        const bool tile = all_tile || g.engine == GemmEngine::kTile ||
                          (g.engine == GemmEngine::kAuto && cnt > kStreamAutoMaxRows);
        items = tile ? (cnt + tile_rows - 1) / tile_rows * tile_nb
                     : (cnt + kStreamItemRows - 1) / kStreamItemRows * stream_nb;
        s_tile[e] = tile;
      }
      const int inc = wave_inclusive_sum(items);
      if (e < E) s_prefix[e] = carry + inc - items;
      carry += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) s_prefix[E] = carry;
  }
}

// The expert owning item t: the last e with s_prefix[e] <= t (s_prefix is non-decreasing, so
// that is the count of such e, minus one). One LDS read and one ballot per 64 experts, the
// whole wave at once, instead of a chain of dependent reads.
__device__ __forceinline__ int expert_of_item(const int* s_prefix, int E, int t) {
  const int lane = lane_id();
  int below = 0;
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    below += __popcll(__ballot(e < E && s_prefix[e] <= t));
  }
  return below - 1;
}

// The items of one workgroup. Workgroup b runs on XCD b % 8, so items are dealt to the XCDs
// in contiguous ranges and the workgroups of an XCD share its L2 for the same experts' rows and
// weights (when the grid is not a multiple of 8: one range, the whole grid). A range is dealt
// in rounds of `step` items (its workgroups); in round k the workgroup takes position
// (slot + k) % step. The rotation hands every workgroup every position in turn, so items of
// unequal cost that recur with a period dividing the step (an expert's short last row block)
// spread over all the workgroups instead of landing on the same few; a round is still the same
// set of consecutive items, and each round is a bijection, so every item runs exactly once.
struct ItemDeal {
  int begin, end, step, slot;
  __device__ __forceinline__ int rounds() const { return (end - begin + step - 1) / step; }
  __device__ __forceinline__ int item(int k) const { return begin + k * step + (slot + k) % step; }
};

__device__ __forceinline__ ItemDeal deal_items(int total) {
  const int nwg = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  if (nwg % 8 != 0) return ItemDeal{0, total, nwg, b};
  const int xcd = b % 8;
  return ItemDeal{static_cast<int>(static_cast<int64_t>(total) * xcd / 8),
                  static_cast<int>(static_cast<int64_t>(total) * (xcd + 1) / 8), nwg / 8, b / 8};
}

// Dynamic dealing (WIDE kernel). The same XCD ranges, but only each workgroup's first item is
// fixed (position `slot` of its range); after that it claims the next item of its range from
// the range's counter (one device atomic a tile, issued when the tile starts and read when it
// ends, so its latency hides behind the tile), and when its range runs out, from the other
// XCDs' ranges in turn. Claims follow item order, so the tiles an XCD runs together stay
// neighbours (shared L2 traffic), while fast workgroups take more items than slow ones: tiles of
// unequal cost (an expert's short last row block) and a range that does not divide evenly no
// longer leave some workgroups with a whole extra tile. Every claim only moves a counter
// forward, so the loop ends; the last workgroup to finish resets the counters to zero.
struct Claims {
  int32_t* sched;  // [0..7] claim counters, [8] finished workgroups
  int total, nranges, home, step, slot;
  __device__ __forceinline__ int begin(int r) const { return static_cast<int>(static_cast<int64_t>(total) * r / nranges); }
  __device__ __forceinline__ int end(int r) const { return static_cast<int>(static_cast<int64_t>(total) * (r + 1) / nranges); }
  __device__ __forceinline__ int range(int ri) const { return (home + ri) % nranges; }
  // claimed index c of range r -> the item (the first `step` items are the fixed first items)
  __device__ __forceinline__ int item(int r, int c) const { return begin(r) + step + c; }
  // thread 0: the next item from range index ri on (advancing ri past exhausted ranges), or -1
  __device__ int claim_from(int& ri) const {
    for (; ri < nranges; ++ri) {
      const int r = range(ri);
      const int t = item(r, atomicAdd(&sched[r], 1));
      if (t < end(r)) return t;
    }
    return -1;
  }
};

__device__ __forceinline__ Claims make_claims(int32_t* sched, int total) {
  const int nwg = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  const int nranges = nwg % 8 == 0 ? 8 : 1;
  return Claims{sched, total, nranges, nranges == 8 ? b % 8 : 0, nwg / nranges, nranges == 8 ? b / 8 : b};
}

// TILE item `local` of an expert with cnt rows -> (row block mt, column block nb): row blocks
// in groups of 4, columns inside a group, so that the consecutive items an XCD runs together
// form 4 x 8 tiles sharing A rows and B columns in its L2.
__device__ __forceinline__ void tile_coords(int local, int cnt, int tile_nb, int& mt, int& nb,
                                            int tile_rows = kTileBM) {
  const int mblocks = (cnt + tile_rows - 1) / tile_rows;
  const int group = local / (4 * tile_nb);
  const int in_group = local - group * 4 * tile_nb;
  const int rows_in_group = min(4, mblocks - group * 4);
  nb = in_group / rows_in_group;
  mt = group * 4 + (in_group - nb * rows_in_group);
}

// kAnyK: K not a multiple of the STREAM chunk (small shapes); the production shapes compile
// without those variants, which keeps the kernel's code (and its cold instruction fetches in
// the one-time prologue) smaller.
// A dual launch's kernel that the routed rows do not select returns at once (GemmArgs).
__device__ __forceinline__ bool dual_skips(const GemmArgs& g, bool wide) {
  return g.dual_rows != nullptr && ((*g.dual_rows >= g.dual_min_rows) != wide);
}

template <bool kGather, bool kSwiglu, bool kAnyK>
__global__ __launch_bounds__(kGemmThreads, 1) void grouped_gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_prefix[kMaxGemmExperts + 1];
  __shared__ int s_tile[kMaxGemmExperts];
  __shared__ int s_count[kMaxGemmExperts];
  __shared__ int s_off[kMaxGemmExperts + 1];
  __shared__ int s_wcnt[kGemmWaves][kMaxGemmExperts];  // in-kernel routing: per-wave counts/bases
  __shared__ int s_tok[kRowTable];
  __shared__ float s_rw[kRowTable];
  __shared__ int s_task[kRowTable];
  __shared__ uint8_t s_ev[kFusedMaxTasks];  // in-kernel routing: expert of each task
  __shared__ TileTables s_tt;                // the current item's scales (epilogue)
  const int E = g.num_experts;
  const RouteArgs& ra = g.route;
  int ntasks = 0;
  bool fused = false;
  if (kSwiglu && g.route_in_kernel) {
    ntasks = effective_tokens(ra.runtime_tokens, ra.host_tokens) * ra.topk;
    fused = g.route_in_kernel == 1 || ntasks <= kFusedMaxTasks;
  }
  // a dual launch: this kernel runs when it routes the live tasks itself (then there are too
  // few rows for WIDE, and the routed-row count is not written yet), else when the routing's
  // row count does not select WIDE
  if (!fused && dual_skips(g, false)) return;
  if (fused) {
    {  // each wave clears its own count row: only that wave adds to it, so no barrier is needed
      const int wave = static_cast<int>(threadIdx.x) / kWave;
      for (int e = lane_id(); e < E; e += kWave) s_wcnt[wave][e] = 0;
    }
    // the route weights stay in the (still unused) dynamic LDS for the first item's row table
    fused_count(ra, ntasks, s_wcnt, s_ev, reinterpret_cast<float*>(smem), blockIdx.x == 0);
    __syncthreads();
    if (threadIdx.x < kWave) {
      fused_scan(E, s_wcnt, s_count, s_off);
      plan_items(g, s_prefix, s_tile, s_count);
    }
    __syncthreads();
    if (blockIdx.x == 0) {  // the routing kernel's outputs that the later stages read
      for (int e = threadIdx.x; e <= E; e += kGemmThreads) ra.offsets[e] = s_off[e];
      for (int e = threadIdx.x; e < E; e += kGemmThreads) {
        ra.counts[e] = s_count[e];
        if (ra.stats != nullptr) ra.stats[e] += s_count[e];
      }
      if (threadIdx.x == 0) {
        ra.meta[0] = s_off[E] < ra.row_cap ? s_off[E] : static_cast<int>(ra.row_cap);
        ra.meta[3] = 0;  // the call's status: no bounded wait on this path
      }
    }
  } else {
    for (int e = threadIdx.x; e <= E; e += kGemmThreads) {
      if (e < E) s_count[e] = g.counts[e];
      s_off[e] = g.offsets[e];
    }
    __syncthreads();
    plan_items(g, s_prefix, s_tile, s_count);
    __syncthreads();
  }
  const int total = s_prefix[E];
  const int tile_nb = (g.n + kTileBN - 1) / kTileBN;
  const bool fast1 = !kAnyK || g.k % (kAChunk / 32) == 0;
  const bool fast2 = !kAnyK || g.k % (kAChunk / 64) == 0;
  const bool fast4 = !kAnyK || g.k % (kAChunk / 128) == 0;
  const ItemDeal deal = deal_items(total);
  // the route weights cached in LDS are valid until the first item's loads overwrite them
  const float* task_w = reinterpret_cast<const float*>(smem);
  bool first_item = true;
  for (int k = 0; k < deal.rounds(); ++k) {
    const int t = deal.item(k);
    if (t >= deal.end) continue;  // the last round's short tail (uniform in the workgroup)
    const float* item_task_w = first_item ? task_w : nullptr;
    first_item = false;
    const int e = expert_of_item(s_prefix, E, t);
    const int local = t - s_prefix[e];
    const int cnt = s_count[e];
    const int off_e = s_off[e];
    if (s_tile[e]) {
      int mt, nb;
      tile_coords(local, cnt, tile_nb, mt, nb);
      RowSrc rs{g.row_token, g.sw.row_weight, 0};
      if (fused) {
        const int r0 = mt * kTileBM;
        fused_rows(ra, ntasks, e, cnt, off_e, s_wcnt, s_ev, item_task_w, r0,
                   nb == 0 ? r0 : 0, nb == 0 ? r0 + kTileBM : 0, 0, 0, s_task, s_tok, s_rw);
        rs = RowSrc{s_tok, s_rw, off_e + r0};
      }
      tile_tile<kGather, kSwiglu>(g, rs, e, off_e + mt * kTileBM, min(kTileBM, cnt - mt * kTileBM),
                                  nb, smem, s_tt);
    } else {
      // An expert's row chunks of one column block (more than one only on the streaming
      // schedule) are neighbouring items, so they run in the same round on the same XCD and
      // read those weight columns from HBM once (through L2).
      const int nch = (cnt + kStreamItemRows - 1) / kStreamItemRows;
      const int nb = local / nch;
      const int mc = local - nb * nch;
      const int mrows = min(kStreamItemRows, cnt - mc * kStreamItemRows);
      const int row0 = off_e + mc * kStreamItemRows;
      RowSrc rs{g.row_token, g.sw.row_weight, 0};
      if (fused) {
        const int r0 = mc * kStreamItemRows;
        fused_rows(ra, ntasks, e, cnt, off_e, s_wcnt, s_ev, item_task_w, r0,
                   nb == 0 ? r0 : 0, nb == 0 ? r0 + kStreamItemRows : 0, 0, 0, s_task, s_tok, s_rw);
        rs = RowSrc{s_tok, s_rw, row0};
      }
      if (mrows > 64) {
        if (fast4) stream_tile<kGather, kSwiglu, 4, true>(g, rs, e, row0, mrows, nb, smem, s_tt);
        else if (kAnyK) stream_tile<kGather, kSwiglu, 4, false>(g, rs, e, row0, mrows, nb, smem, s_tt);
      } else if (mrows > 32) {
        if (fast2) stream_tile<kGather, kSwiglu, 2, true>(g, rs, e, row0, mrows, nb, smem, s_tt);
        else if (kAnyK) stream_tile<kGather, kSwiglu, 2, false>(g, rs, e, row0, mrows, nb, smem, s_tt);
      } else {
        if (fast1) stream_tile<kGather, kSwiglu, 1, true>(g, rs, e, row0, mrows, nb, smem, s_tt);
        else if (kAnyK) stream_tile<kGather, kSwiglu, 1, false>(g, rs, e, row0, mrows, nb, smem, s_tt);
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ decode pipeline
// GEMM1 (with the in-kernel routing), the requant and GEMM2 of the streaming engine in one
// launch, so that a group of rows goes on to GEMM2 as soon as its own GEMM1 items are done,
// instead of after the slowest XCD's last GEMM1 item, and without the requant's and GEMM2's
// launches and prologues.
//
// Work: the routed rows are cut into groups (an expert's rows in chunks of kStreamRows); a group
// has n1 GEMM1 items and n2 GEMM2 items (512-column blocks). The groups are dealt to the XCDs in
// contiguous ranges, and the workgroups of an XCD -- found by the hardware XCD id, not by launch
// order -- claim its queue in order: every GEMM1 item of its groups, then their GEMM2 items. A
// claim goes out one item ahead, so its latency hides behind an item.
//
// Hand-off, inside the XCD, whose CUs share its L2 (the per-CU L1 is write-through): a GEMM1
// item waits for its bf16 SwiGLU stores (vmcnt 0) and counts itself done for its group. A GEMM2
// item issues its first weight steps, polls until its group's count is complete, invalidates
// its CU's L1 and requantizes the group's rows from L2 straight into its LDS A buffers (the
// requant kernel's arithmetic, so the same bits; the group's first GEMM2 item also writes act
// and amax out). Every GEMM1 item is claimed before any GEMM2 item of its XCD, and a GEMM1 item
// waits on nothing, so every wait ends; a wait is also bounded (kPipeSpinLimit polls), and one
// that runs out is counted (the launch's last workgroup leaves the count in meta[3], the call's
// status) instead of hanging. The workgroup that finishes last runs the
// queue of any XCD that no workgroup ran (none when the launch covers the chip), alone and
// start to end.
//
// Combine (PipeArgs::y set): a GEMM2 item stores its partial rows device-coherent (sc1: written
// through the XCD's L2, which other XCDs do not see), drains them and counts itself done for its
// expert. A workgroup out of items combines its share of the tokens, one wave a token: for each
// routed slot (the task's expert from the routing's LDS table) it waits until the expert's
// GEMM1 items are done (its rows' output_index entries are written, also device-coherent) and
// loads the row, then until the expert's GEMM2 items are done, and reads the partial rows with
// device-coherent loads. Every GEMM2 item is claimed by a workgroup of its XCD, or by the last
// workgroup for an XCD without any, so every wait ends. The workgroup that leaves last sets the
// counters back to zero.
__device__ __forceinline__ int hw_xcc_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

// This wave's outstanding memory operations (the stores a hand-off publishes) are complete.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Later loads of this CU miss its L1 (they read the XCD's L2, where the producer's stores are).
__device__ __forceinline__ void l1_invalidate() { asm volatile("buffer_inv sc0" ::: "memory"); }

// Thread-level poll (a vector atomic load: lane-divergent code) until *c >= target, at most
// `limit` polls (false: it ran out).
__device__ __forceinline__ bool wait_count(const int32_t* c, int target, int limit) {
  for (int i = 0; i < limit; ++i) {
    if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) return true;
    __builtin_amdgcn_s_sleep(2);
  }
  return false;
}

// One 16-byte piece at byte offset off of a buffer, device-coherent (sc1: an L2 line that another
// XCD wrote is not served stale).
__device__ __forceinline__ uint4 ld16_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16 /* sc1 */);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// The combine of token t in the decode pipeline (one wave, whole rows of H <= 64 * 8 * 8
// columns): the slot-ordered fp32 sum of its routed slots' partial rows from +0, bf16 RNE (the
// combine kernel's arithmetic, so the same bits); a token without routed slots gets zeros.
constexpr int kPipeCombineV = 8;  // 16-byte column groups per lane

__device__ void pipe_combine_token(const PipeArgs& p, int64_t t, const uint8_t* s_ev,
                                   const int* s_gprefix, int n1, int n2, const int32_t* done1,
                                   const int32_t* done2, __amdgpu_buffer_rsrc_t part) {
  constexpr int V = kPipeCombineV;
  const RouteArgs& ra = p.g1.route;
  const int lane = lane_id();
  const int hidden = p.g2.n;
  const int nvec = hidden >> 3;
  int row = -1;
  if (lane < ra.topk) {
    const int64_t task = t * ra.topk + lane;
    const int ev = s_ev[task];
    if (ev != 255) {
      bool ok = true;
      for (int grp = s_gprefix[ev]; grp < s_gprefix[ev + 1]; ++grp)
        ok = ok && wait_count(&done1[grp], n1, p.spin_limit);
      row = __hip_atomic_load(&ra.output_index[task], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = ok && wait_count(&done2[ev * kPipeDone2Stride], n2 * (s_gprefix[ev + 1] - s_gprefix[ev]),
                            p.spin_limit);
      if (!ok) atomicAdd(&p.pipe[kPipeFailAt], 1);
    }
  }
  float sum[V][8];
#pragma unroll
  for (int j = 0; j < V; ++j)
#pragma unroll
    for (int q = 0; q < 8; ++q) sum[j][q] = 0.0f;
  // the routed slots in ascending order, two at a time (their loads go out together)
  constexpr int kSlots = 2;
  for (uint64_t m = __ballot(row >= 0); m != 0;) {
    uint4 pv[kSlots][V];
    bool has[kSlots];
#pragma unroll
    for (int b = 0; b < kSlots; ++b) {
      has[b] = m != 0;  // wave-uniform (a ballot)
      const int s = has[b] ? __ffsll(static_cast<unsigned long long>(m)) - 1 : 0;
      m &= m - 1;
      const int r = __shfl(row, s, kWave);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int v = j * kWave + lane;
        pv[b][j] = has[b] && v < nvec ? ld16_coherent(part, (r * hidden + v * 8) * 2) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int b = 0; b < kSlots; ++b) {
      if (!has[b]) break;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const uint32_t words[4] = {pv[b][j].x, pv[b][j].y, pv[b][j].z, pv[b][j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sum[j][2 * q] += bf16_to_f32(words[q] & 0xffff);
          sum[j][2 * q + 1] += bf16_to_f32(words[q] >> 16);
        }
      }
    }
  }
  uint4* yrow = reinterpret_cast<uint4*>(p.y + t * hidden);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int v = j * kWave + lane;
    if (v < nvec)
      yrow[v] = make_uint4(pack_bf16x2(sum[j][0], sum[j][1]), pack_bf16x2(sum[j][2], sum[j][3]),
                           pack_bf16x2(sum[j][4], sum[j][5]), pack_bf16x2(sum[j][6], sum[j][7]));
  }
}

// Wave 0: s_gprefix[0..E] = exclusive prefix of the experts' groups (chunks of kStreamRows rows).
__device__ void plan_groups(int E, const int* s_count, int* s_gprefix) {
  const int lane = lane_id();
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    const int n = e < E ? (s_count[e] + kStreamRows - 1) / kStreamRows : 0;
    const int inc = wave_inclusive_sum(n);
    if (e < E) s_gprefix[e] = carry + inc - n;
    carry += __shfl(inc, kWave - 1, kWave);
  }
  if (lane == 0) s_gprefix[E] = carry;
}

// The requant of rows [row0, row0 + mrows) of GEMM1's bf16 output y into the LDS A chunk buffers
// of a STREAM GEMM2 tile of MT 32-row tiles (stream_tile's chunk layout; K = I in one chunk for
// MT = 1, two for MT = 2): the row's amax, inv = 448 / max(amax, 1e-4), then 16 e4m3 codes per
// LDS piece -- the requant kernel's arithmetic, so the same bits. The amax is the max of the
// row's 64 partial maxima that GEMM1's epilogue stored (one per 64-column block, exact), eight
// lanes a row. The row scale a/448 goes straight into the tile's LDS scale table (s_xs); with
// write_act the rows' act, act_scale and amax also go out. The y pieces go out kStageBatch at a
// time, the first batch together with the maxima; rows past mrows are neither loaded nor
// quantized (their LDS rows feed only accumulator rows that are never stored).
constexpr int kStageBatch = 4;

template <int MT>
__device__ void stage_rows_from_y(const PipeArgs& p, int row0, int mrows, bool write_act,
                                  uint8_t* smem, float* s_inv, float* s_xs) {
  constexpr int kc = kAChunk / (32 * MT);
  constexpr int kUnits = 2 * 2048 / kStreamUnit;  // partial maxima per row (I = 2048)
  static_assert(kStreamRows == kGemmWaves * kWave / 8, "eight lanes per row cover the group");
  static_assert(kALoads % kStageBatch == 0, "whole batches");
  const int inter = p.g1.sw.inter;
  const int nchunks = inter / kc;
  const int tid = opaque_tid();
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const uint16_t* y = p.g1.sw.y;
  const int r8 = tid >> 3;
  float4 pm[kUnits / 32];
#pragma unroll
  for (int j = 0; j < kUnits / 32; ++j) pm[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (r8 < mrows) {
    const float4* src = reinterpret_cast<const float4*>(
        p.g1.row_pmax + static_cast<int64_t>(row0 + r8) * kUnits + (tid & 7) * (kUnits / 8));
#pragma unroll
    for (int j = 0; j < kUnits / 32; ++j) pm[j] = src[j];
  }
  // batch b of chunk c: pieces i = b * kStageBatch + h; piece i of a lane holds LDS bytes
  // (i * 8 + wave) * 1024 + lane * 16 of the chunk buffer (row r, swizzled piece): 16 channels,
  // 32 bytes of y
  uint4 v[kStageBatch][2];
  auto load_batch = [&](int c, int b) {
#pragma unroll
    for (int h = 0; h < kStageBatch; ++h) {
      const int pos = ((b * kStageBatch + h) * kGemmWaves + wave) * 1024 + lane * 16;
      const int r = pos / kc;
      const int off = c * kc + swizzle_piece((pos - r * kc) >> 4, r) * 16;
      if (r < mrows) {
        const uint4* src = reinterpret_cast<const uint4*>(y + static_cast<int64_t>(row0 + r) * inter + off);
        v[h][0] = src[0];
        v[h][1] = src[1];
      }
    }
  };
  auto lo = [](uint32_t w) { return bf16_to_f32(static_cast<uint16_t>(w & 0xffff)); };
  auto hi = [](uint32_t w) { return bf16_to_f32(static_cast<uint16_t>(w >> 16)); };
  load_batch(0, 0);
  {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kUnits / 32; ++j) m = fmaxf(fmaxf(fmaxf(m, pm[j].x), fmaxf(pm[j].y, pm[j].z)), pm[j].w);
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if ((tid & 7) == 0 && r8 < mrows) {
      s_inv[r8] = kE4m3Max / fmaxf(m, kAmaxFloor);
      s_xs[r8] = fmaxf(m, kAmaxFloor) / kE4m3Max;
      if (write_act) {
        p.act_scale[row0 + r8] = fmaxf(m, kAmaxFloor) / kE4m3Max;
        p.amax[row0 + r8] = m;
      }
    }
  }
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    for (int b = 0; b < kALoads / kStageBatch; ++b) {
      if (c > 0 || b > 0) load_batch(c, b);
#pragma unroll
      for (int h = 0; h < kStageBatch; ++h) {
        const int i = b * kStageBatch + h;
        const int pos = (i * kGemmWaves + wave) * 1024 + lane * 16;
        const int r = pos / kc;
        int4 q = make_int4(0, 0, 0, 0);  // rows past mrows: never stored
        if (r < mrows) {
          const float inv = s_inv[r];
          const uint4 a = v[h][0], b2 = v[h][1];
          q.x = static_cast<int>(pack_e4m3x4(lo(a.x) * inv, hi(a.x) * inv, lo(a.y) * inv, hi(a.y) * inv));
          q.y = static_cast<int>(pack_e4m3x4(lo(a.z) * inv, hi(a.z) * inv, lo(a.w) * inv, hi(a.w) * inv));
          q.z = static_cast<int>(pack_e4m3x4(lo(b2.x) * inv, hi(b2.x) * inv, lo(b2.y) * inv, hi(b2.y) * inv));
          q.w = static_cast<int>(pack_e4m3x4(lo(b2.z) * inv, hi(b2.z) * inv, lo(b2.w) * inv, hi(b2.w) * inv));
          if (write_act) {
            const int off = c * kc + swizzle_piece((pos - r * kc) >> 4, r) * 16;
            *reinterpret_cast<int4*>(p.act + static_cast<int64_t>(row0 + r) * inter + off) = q;
          }
        }
        *reinterpret_cast<int4*>(smem + (c & 1) * kAChunk + wave * 1024 + lane * 16 + i * kGemmWaves * 1024) = q;
      }
    }
  }
}

__global__ __launch_bounds__(kGemmThreads, 1) void decode_pipeline_kernel(PipeArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_gprefix[kMaxGemmExperts + 1];
  __shared__ int s_count[kMaxGemmExperts];
  __shared__ int s_off[kMaxGemmExperts + 1];
  __shared__ int s_wcnt[kGemmWaves][kMaxGemmExperts];
  __shared__ int s_tok[kRowTable];
  __shared__ float s_rw[kRowTable];
  __shared__ int s_task[kRowTable];
  __shared__ uint8_t s_ev[kFusedMaxTasks];
  __shared__ TileTables s_tt;
  __shared__ float s_inv[kStreamRows];
  __shared__ int s_word;  // thread 0 -> the workgroup
  const GemmArgs& g1 = p.g1;
  const GemmArgs& g2 = p.g2;
  const RouteArgs& ra = g1.route;
  const int E = g1.num_experts;
  int32_t* const claims = p.pipe;  // XCD x's counter at claims[x * kPipeLine]
  int32_t* const finish = p.pipe + kPipeFinishAt;
  int32_t* const done1 = p.pipe + kPipeDone1At;  // [groups]
  int32_t* const done2 = p.pipe + kPipeDone2At;  // [experts]
  const int hw = hw_xcc_id();
  const int home = hw & (kPipeXcds - 1);
  int x = home;
  // thread 0: the first claim (its latency hides behind the routing); a workgroup's home XCD
  // counter is nonzero from then on, which is how the last workgroup finds XCDs without any
  int pending = 0;
  if (threadIdx.x == 0) pending = atomicAdd(&claims[x * kPipeLine], 1);
  const int ntasks = effective_tokens(ra.runtime_tokens, ra.host_tokens) * ra.topk;
  {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    for (int e = lane_id(); e < E; e += kWave) s_wcnt[wave][e] = 0;
  }
  fused_count(ra, ntasks, s_wcnt, s_ev, reinterpret_cast<float*>(smem), blockIdx.x == 0);
  __syncthreads();
  if (threadIdx.x < kWave) {
    fused_scan(E, s_wcnt, s_count, s_off);
    plan_groups(E, s_count, s_gprefix);
  }
  __syncthreads();
  if (blockIdx.x == 0) {  // the routing outputs that the later stages read
    for (int e = threadIdx.x; e <= E; e += kGemmThreads) ra.offsets[e] = s_off[e];
    for (int e = threadIdx.x; e < E; e += kGemmThreads) {
      ra.counts[e] = s_count[e];
      if (ra.stats != nullptr) ra.stats[e] += s_count[e];
    }
    if (threadIdx.x == 0) {
      ra.meta[0] = s_off[E] < ra.row_cap ? s_off[E] : static_cast<int>(ra.row_cap);
      p.meta[1] = 0;  // the 8-wave GEMM1
      if (p.direct_flag != nullptr) *p.direct_flag = 0;
      if (hw >= kPipeXcds) atomicAdd(&p.pipe[kPipeFailAt], 1);  // an XCD id this launch does not expect
    }
  }
  // more groups than counters (the host's task bound rules it out): flagged, and no items
  const bool too_many = s_gprefix[E] > kMaxPipeGroups;
  if (too_many && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&p.pipe[kPipeFailAt], 1);
  const int G = too_many ? 0 : s_gprefix[E];
  const int n1 = stream_blocks(g1), n2 = stream_blocks(g2);
  const float* task_w = reinterpret_cast<const float*>(smem);  // valid until the first item's loads
  bool first_item = true;
  int present = -1;  // the last workgroup: XCDs that had workgroups (bit mask)
  int orphan = -1;   // the last workgroup: the XCD queue it runs
  for (;;) {
    if (threadIdx.x == 0) s_word = pending;
    __syncthreads();
    const int t = s_word;
    __syncthreads();
    const int gb = static_cast<int>(static_cast<int64_t>(G) * x / kPipeXcds);
    const int ng = static_cast<int>(static_cast<int64_t>(G) * (x + 1) / kPipeXcds) - gb;
    if (t >= (n1 + n2) * ng) {
      if (present < 0) {
        // count this workgroup finished (after its last claim was answered); the last one
        // learns which XCDs had workgroups: those whose claim counter moved
        if (threadIdx.x == 0) {
          const bool is_last = atomicAdd(finish, 1) == static_cast<int>(gridDim.x) - 1;
          int mask = -1;
          if (is_last) {
            mask = 0;
            for (int q = 0; q < kPipeXcds; ++q)
              if (__hip_atomic_load(&claims[q * kPipeLine], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
                mask |= 1 << q;
          }
          s_word = mask;
        }
        __syncthreads();
        present = s_word;
        __syncthreads();
        if (present < 0) break;
      }
      // every other workgroup has finished: the queues of XCDs without workgroups, whole
      do ++orphan; while (orphan < kPipeXcds && ((present >> orphan) & 1));
      if (orphan >= kPipeXcds) break;
      x = orphan;
      if (threadIdx.x == 0) pending = atomicAdd(&claims[x * kPipeLine], 1);
      continue;
    }
    if (threadIdx.x == 0) pending = atomicAdd(&claims[x * kPipeLine], 1);  // the next claim, one item ahead
    const bool gemm1 = t < n1 * ng;
    const int local = gemm1 ? t : t - n1 * ng;
    const int per = gemm1 ? n1 : n2;
    const int grp = gb + local / per;
    const int nb = local - (local / per) * per;
    const int e = expert_of_item(s_gprefix, E, grp);
    const int r0 = (grp - s_gprefix[e]) * kStreamRows;
    const int cnt = s_count[e];
    const int off_e = s_off[e];
    const int mrows = min(kStreamRows, cnt - r0);
    const int row0 = off_e + r0;
    if (gemm1) {
      // the weights go out first; then the item's rows are ranked into the LDS row table
      const float* item_w = first_item ? task_w : nullptr;
      const auto rank_rows = [&]() {
        fused_rows(ra, ntasks, e, cnt, off_e, s_wcnt, s_ev, item_w, r0, nb == 0 ? r0 : 0,
                   nb == 0 ? r0 + kStreamRows : 0, 0, 0, s_task, s_tok, s_rw);
      };
      const RowSrc rs{s_tok, s_rw, row0};
      if (mrows > 32) stream_tile<true, true, 2, true, true, false, true, true>(g1, rs, e, row0, mrows, nb, smem, s_tt, rank_rows);
      else stream_tile<true, true, 1, true, true, false, true, true>(g1, rs, e, row0, mrows, nb, smem, s_tt, rank_rows);
      vm_drain();  // this wave's y stores are in L2
      __syncthreads();
      if (threadIdx.x == 0) atomicAdd(&done1[grp], 1);
    } else {
      // the weights go out first; then the group's rows, requantized from y into LDS
      const auto stage_rows = [&]() {
        if (threadIdx.x == 0 && !wait_count(&done1[grp], n1, p.spin_limit)) atomicAdd(&p.pipe[kPipeFailAt], 1);
        __syncthreads();
        l1_invalidate();
        if (mrows > 32) stage_rows_from_y<2>(p, row0, mrows, nb == 0, smem, s_inv, s_tt.xs);
        else stage_rows_from_y<1>(p, row0, mrows, nb == 0, smem, s_inv, s_tt.xs);
        __syncthreads();
      };
      const RowSrc rs{nullptr, nullptr, 0};
      if (mrows > 32)
        stream_tile<false, false, 2, true, true, true, false, true>(g2, rs, e, row0, mrows, nb, smem, s_tt, stage_rows);
      else
        stream_tile<false, false, 1, true, true, true, false, true>(g2, rs, e, row0, mrows, nb, smem, s_tt, stage_rows);
      vm_drain();  // this wave's partial rows are written through to the device-coherent level
      __syncthreads();
      if (threadIdx.x == 0) atomicAdd(&done2[e * kPipeDone2Stride], 1);
    }
    first_item = false;
    __syncthreads();
  }
  if (p.y != nullptr && !too_many) {
    // the combine: token i goes to wave (i / gridDim.x) % 8 of workgroup i % gridDim.x, so the
    // tokens spread over all workgroups (each wave's tokens are independent of the others')
    const int tokens = effective_tokens(ra.runtime_tokens, ra.host_tokens);
    const int64_t part_bytes = static_cast<int64_t>(ra.row_cap) * g2.n * 2;
    const __amdgpu_buffer_rsrc_t part = __builtin_amdgcn_make_buffer_rsrc(
        g2.c, 0, static_cast<int>(part_bytes < 0x7fffffff ? part_bytes : 0x7fffffff), 0x00020000);
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    for (int64_t t = blockIdx.x + static_cast<int64_t>(wave) * gridDim.x; t < tokens;
         t += static_cast<int64_t>(gridDim.x) * kGemmWaves)
      pipe_combine_token(p, t, s_ev, s_gprefix, n1, n2, done1, done2, part);
  }
  // the workgroup that leaves last (every other one has made its last counter access): the
  // count of waits that ran out into meta[3] (the call's status), the counters back to zero
  // for the next launch. Each wave's counter atomics are complete (vmcnt) before its
  // workgroup counts itself out, so the last one reads every failure.
  vm_drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = atomicAdd(p.pipe + kPipeExitAt, 1) == static_cast<int>(gridDim.x) - 1;
    if (last) p.meta[3] = __hip_atomic_load(p.pipe + kPipeFailAt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_word = last ? 1 : 0;
  }
  __syncthreads();
  if (s_word != 0) {
    for (int i = threadIdx.x; i < kPipeHeader + G; i += kGemmThreads) p.pipe[i] = 0;
    for (int i = threadIdx.x; i < E; i += kGemmThreads) done2[i * kPipeDone2Stride] = 0;
  }
}

// Persistent dispatcher of the WIDE engine: every expert's rows as BM x 256 tiles, items dealt
// to the XCDs in contiguous ranges like the 8-wave dispatcher's.
template <bool kGather, bool kSwiglu, int BM>
__global__ __launch_bounds__(kWideThreads, WideShape<BM>::kWavesPerSimd) void wide_gemm_kernel(GemmArgs g) {
  if (dual_skips(g, true)) return;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_prefix[kMaxGemmExperts + 1];
  __shared__ int s_tile[kMaxGemmExperts];
  __shared__ int s_count[kMaxGemmExperts];
  __shared__ int s_off[kMaxGemmExperts + 1];
  const int E = g.num_experts;
  for (int e = threadIdx.x; e <= E; e += kWideThreads) {
    if (e < E) s_count[e] = g.counts[e];
    s_off[e] = g.offsets[e];
  }
  __syncthreads();
  plan_items(g, s_prefix, s_tile, s_count, true, BM);
  __syncthreads();
  const int total = s_prefix[E];
  const int tile_nb = (g.n + kTileBN - 1) / kTileBN;
  const RowSrc rs{g.row_token, g.sw.row_weight, 0};
  auto run_item = [&](int t, const auto& before_epilogue) {
    const int e = expert_of_item(s_prefix, E, t);
    const int cnt = s_count[e];
    int mt, nb;
    tile_coords(t - s_prefix[e], cnt, tile_nb, mt, nb, BM);
    const int mrows = min(BM, cnt - mt * BM);
    const int row0 = s_off[e] + mt * BM;
    if (BM == 256 && mrows > 128)
      wide_tile<kGather, kSwiglu, BM, (BM == 256 ? 8 : 4)>(g, rs, e, row0, mrows, nb, smem, before_epilogue);
    else if (mrows > 64)
      wide_tile<kGather, kSwiglu, BM, 4>(g, rs, e, row0, mrows, nb, smem, before_epilogue);
    else if (mrows > 32)
      wide_tile<kGather, kSwiglu, BM, 2>(g, rs, e, row0, mrows, nb, smem, before_epilogue);
    else
      wide_tile<kGather, kSwiglu, BM, 1>(g, rs, e, row0, mrows, nb, smem, before_epilogue);
  };
  // One item at a time from the static deal or from the claims. Claiming only pays when a
  // workgroup has few items (the last round's granularity is then a large share of its work;
  // 24.7K routed rows: 7 items a workgroup, 5% faster); with many it measured slower (196K rows,
  // 49 items: 1% slower; 49K Zipf rows, 13 items: 1% slower) -- the lockstep rounds of the static
  // deal keep an XCD's concurrent tiles on the same rows and weights, and at those sizes the
  // chip is power-bound, so idle workgroups cost less than the looser L2 sharing.
  constexpr int kClaimMaxItemsPerWg = 10;
  const bool dynamic =
      g.sched != nullptr && total <= kClaimMaxItemsPerWg * static_cast<int>(gridDim.x);
  const ItemDeal deal = deal_items(total);
  const Claims cl = make_claims(g.sched, total);
  __shared__ int s_item;
  int k = 0;   // static: the round
  int ri = 0;  // dynamic, thread 0: index of the range it claims from
  if (threadIdx.x == 0 && dynamic) {
    const int first = cl.begin(cl.home) + cl.slot;
    s_item = first < cl.end(cl.home) ? first : cl.claim_from(ri);
  }
  __syncthreads();
  while (true) {
    int t;
    if (dynamic) {
      t = s_item;
    } else {
      for (t = -1; k < deal.rounds() && t < 0; ++k) {
        const int c = deal.item(k);
        t = c < deal.end ? c : -1;  // the last round's short tail
      }
    }
    if (t < 0) break;
    // thread 0: the claim for the item after this one, issued when the tile's MFMAs are done
    // (its latency hides behind the epilogue; issued at the tile's start, its result stayed live
    // through the tile and was spilled, with a wait for every memory operation in flight)
    int pending = 0;
    run_item(t, [&]() {
      if (dynamic && threadIdx.x == 0 && ri < cl.nranges) pending = atomicAdd(&g.sched[cl.range(ri)], 1);
    });
    if (dynamic && threadIdx.x == 0) {
      int next = -1;
      if (ri < cl.nranges) {
        const int r = cl.range(ri);
        next = cl.item(r, pending);
        if (next >= cl.end(r)) {
          ++ri;
          next = cl.claim_from(ri);
        }
      }
      s_item = next;  // read after the barrier; rewritten only after the next tile's barriers
    }
    __syncthreads();
  }
  if (g.zf.y != nullptr && !dynamic) {
    // out of tiles: the zero y rows of tokens without a valid routed slot, a claimed chunk of
    // kZeroFillTokens tokens at a time (a wave a token), while other workgroups still run tiles
    // (z.idle counts the workgroups out of tiles); the combine writes the chunks left. Only
    // with the static deal (many tiles a workgroup): with claimed tiles the idle end is short,
    // and the zero rows' writes slowed the last tiles by more than the combine saved (c2: +28 us
    // per layer; c3: -60 us).
    const ZeroFill& z = g.zf;
    const int tokens = effective_tokens(z.runtime_tokens, z.host_tokens);
    const int nchunks = (tokens + kZeroFillTokens - 1) / kZeroFillTokens;
    const int lane = lane_id(), wave = static_cast<int>(threadIdx.x) / kWave;
    const int nvec = z.hidden >> 3;
    if (threadIdx.x == 0) atomicAdd(z.idle, 1);
    for (;;) {
      __syncthreads();  // every thread has read s_item
      if (threadIdx.x == 0) {
        const int idle = __hip_atomic_load(z.idle, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_item = idle >= static_cast<int>(gridDim.x) ? nchunks : atomicAdd(z.claim, 1);
      }
      __syncthreads();
      const int c = s_item;
      if (c >= nchunks) break;
      const int t_end = min(tokens, (c + 1) * kZeroFillTokens);
      for (int t = c * kZeroFillTokens + wave; t < t_end; t += kWideWaves) {
        const int v = lane < z.topk ? z.output_index[static_cast<int64_t>(t) * z.topk + lane] : -1;
        if (__ballot(v >= 0) != 0) continue;
        i32x4* row = reinterpret_cast<i32x4*>(z.y + static_cast<int64_t>(t) * z.hidden);
        for (int i = lane; i < nvec; i += kWave) __builtin_nontemporal_store(i32x4{0, 0, 0, 0}, row + i);
      }
    }
  }
  if (dynamic && threadIdx.x == 0) {  // every claim of this workgroup is done: count it out
    if (atomicAdd(&g.sched[8], 1) == static_cast<int>(gridDim.x) - 1) {
      for (int r = 0; r < 8; ++r) atomicExch(&g.sched[r], 0);
      atomicExch(&g.sched[8], 0);
    }
  }
}

// The dynamic-LDS limit of kernel K raised to `bytes` (above the default) once per device of
// the process (the attribute is set for the current device; a bit per device id below 64).
template <auto K>
hipError_t ensure_dynamic_lds(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const uint64_t bit = dev >= 0 && dev < 64 ? (1ull << dev) : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(K), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err == hipSuccess && bit != 0) done.fetch_or(bit, std::memory_order_release);
  return err;
}

template <bool kGather, bool kSwiglu, int BM>
hipError_t launch_wide(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  using W = WideShape<BM>;
  {  // the dynamic LDS (up to 104 KB) exceeds the default limit
    const hipError_t err = ensure_dynamic_lds<&wide_gemm_kernel<kGather, kSwiglu, BM>>(W::kSmemBytes);
    if (err != hipSuccess) return err;
  }
  const int64_t bound =
      (static_cast<int64_t>(max_rows) / BM + g.num_experts) * ((g.n + kTileBN - 1) / kTileBN);
  int64_t grid = static_cast<int64_t>(num_cus) * W::kWavesPerSimd;  // workgroups a CU: 1 or 2
  if (grid > bound) grid = bound;
  return launch_kernel(wide_gemm_kernel<kGather, kSwiglu, BM>, dim3(static_cast<unsigned>(grid)),
                       dim3(kWideThreads), W::kSmemBytes, stream, g);
}

template <bool kGather, bool kSwiglu, bool kAnyK>
hipError_t launch_engines_k(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  {  // the 128 KB of dynamic LDS exceeds the default limit
    const hipError_t err = ensure_dynamic_lds<&grouped_gemm_kernel<kGather, kSwiglu, kAnyK>>(kSmemBytes);
    if (err != hipSuccess) return err;
  }
  // upper bound of the work items over any split of max_rows rows into the experts
  const int64_t stream_nb = (g.n / kStreamUnit + kGemmWaves - 1) / kGemmWaves;
  const int64_t stream_items = (static_cast<int64_t>(max_rows) / kStreamItemRows + g.num_experts) * stream_nb;
  const int64_t tile_items =
      (static_cast<int64_t>(max_rows) / kTileBM + g.num_experts) * ((g.n + kTileBN - 1) / kTileBN);
  const int64_t bound = g.engine == GemmEngine::kStream ? stream_items
                        : g.engine == GemmEngine::kTile ? tile_items
                                                        : std::max(stream_items, tile_items);
  int64_t grid = num_cus;  // one 8-wave workgroup per CU
  if (grid > bound) grid = bound;
  return launch_kernel(grouped_gemm_kernel<kGather, kSwiglu, kAnyK>, dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
}

template <bool kGather, bool kSwiglu>
hipError_t launch_engines(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  return g.k % (kAChunk / 32) == 0 ? launch_engines_k<kGather, kSwiglu, false>(g, max_rows, num_cus, stream)
                                    : launch_engines_k<kGather, kSwiglu, true>(g, max_rows, num_cus, stream);
}

}  // namespace

int gemm_route_max_tasks() { return kFusedMaxTasks; }
int gemm_route_max_experts() { return kFusedMaxExperts; }

// Many rows per expert on average: every expert as WIDE tiles (one launch, no per-expert engine
// choice). More tasks than the in-kernel routing takes, so the two never meet; the choice
// depends only on the shape and the row bound, so separate stage calls agree on it.
bool gemm_wide_selected(const GemmArgs& g, int max_rows) {
  return g.engine != GemmEngine::kStream && g.k % (2 * kWideBK) == 0 && g.n % kStreamUnit == 0 &&
         max_rows > kFusedMaxTasks &&
         static_cast<int64_t>(max_rows) >= static_cast<int64_t>(kWideMinRowsPerExpert) * g.num_experts;
}

bool gemm_shape_supported(int n, int k) {
  return n > 0 && k > 0 && n % 128 == 0 && k % 128 == 0;
}

// Full WIDE tile heights. 256 rows (one workgroup a CU) for both GEMMs: with 128-row tiles and
// two workgroups a CU, GEMM1 (weights read twice as often) ran 1.33x slower at the 196K-row
// prefill; GEMM2 ran 7% faster at 24.7K rows but slower at 196K rows, where it also left the
// next layer's GEMM1 2% slower (measured on one box, builds alternated).
constexpr int kWideBM1 = 256;
constexpr int kWideBM2 = 256;

int gemm_wide_min_rows(int num_experts) {
  return std::max(kFusedMaxTasks + 1, kWideMinRowsPerExpert * num_experts);
}

// Eager calls whose row bound selects WIDE only by a small margin: the routed rows may be far
// fewer (an EP share keeps ~1/8 of its slots), so both kernels go out and the routing's largest
// expert row count chooses on the device -- the 8-wave kernels while every expert has at most
// 128 rows (one STREAM item a column block), WIDE from 129.
// Measured (whole eager layers after a read-only cache flush) at T = 256..576 a rank (256 global
// experts, top-6): 188-202 us on the 8-wave kernels (one 128-row item per expert and column
// block: 256 items, one round) against 230-248 us on WIDE. Streaming experts of up to 256 rows
// (two items) and going WIDE only past that was within -4..+3% of this choice at T = 640..1024.
// Auto schedules only (an engine set by the caller keeps its kernels); from 8 x 128 tasks an
// expert (an EP share of 1/8 then routes 128 rows an expert on average, so some expert has
// more) the bound selects WIDE directly (no launches that return at once).
constexpr int kEagerDualMinLargest = kStreamAutoMaxRows + 1;
int gemm_eager_dual_min_largest() { return kEagerDualMinLargest; }
bool gemm_eager_dual(const GemmArgs& g, int max_rows) {
  return g.engine == GemmEngine::kAuto && gemm_wide_selected(g, max_rows) &&
         static_cast<int64_t>(max_rows) < 8ll * kStreamAutoMaxRows * g.num_experts;
}

// The decode pipeline needs the streaming engine's full-chunk shapes for both GEMMs (GEMM2's
// K = I in at most two chunks, staged whole by the requant), GEMM1's in-kernel routing, and
// the whole MI355X (8 XCDs of 32 CUs: its queues are the hardware XCD ids).
bool decode_pipeline_supported(const GemmArgs& g1, const GemmArgs& g2, int num_cus) {
  return num_cus == kPipeXcds * 32 && g1.engine != GemmEngine::kTile && g2.engine != GemmEngine::kTile &&
         g1.route_in_kernel == 1 && g1.sw.enabled && g1.num_experts <= kFusedMaxExperts &&
         g1.k % (kAChunk / 32) == 0 && g2.k == kAChunk / 32 && g1.n == 2 * g1.sw.inter &&
         g2.k == g1.sw.inter && g1.n % (kStreamUnit * kGemmWaves) == 0 &&
         g2.n % (kStreamUnit * kGemmWaves) == 0 && g1.row_token != nullptr && g2.row_token == nullptr &&
         g1.dual_rows == nullptr && g2.dual_rows == nullptr && g2.y_direct == nullptr;
}

hipError_t launch_decode_pipeline(const PipeArgs& p, int num_cus, hipStream_t stream) {
  if (!decode_pipeline_supported(p.g1, p.g2, num_cus) || p.pipe == nullptr || p.g1.row_pmax == nullptr ||
      p.act != p.g2.a ||
      p.act_scale != p.g2.a_scale || p.g2.lda != p.g1.sw.inter)
    return hipErrorInvalidValue;
  const hipError_t err = ensure_dynamic_lds<&decode_pipeline_kernel>(kSmemBytes);
  if (err != hipSuccess) return err;
  return launch_kernel(decode_pipeline_kernel, dim3(static_cast<unsigned>(num_cus)), dim3(kGemmThreads),
                       kSmemBytes, stream, p);
}

hipError_t launch_grouped_gemm(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream,
                               const int32_t* rows_on_device, bool route_small_in_kernel,
                               int dual_min_rows) {
  if (max_rows <= 0) return hipSuccess;
  if (g.num_experts > kMaxGemmExperts || g.dual_rows != nullptr) return hipErrorInvalidValue;
  const bool wide = gemm_wide_selected(g, max_rows);
  if (wide && g.route_in_kernel) return hipErrorInvalidValue;
  // direct writes to y: the WIDE GEMM2 epilogue only
  if (g.y_direct != nullptr && (!wide || g.sw.enabled || g.row_dest == nullptr || g.direct_flag == nullptr))
    return hipErrorInvalidValue;
  if (g.sw.enabled && (g.row_token == nullptr || g.n != 2 * g.sw.inter)) return hipErrorInvalidValue;
  if (!g.sw.enabled && g.row_token != nullptr) return hipErrorInvalidValue;
  // the 8-wave kernel routes the live tasks itself when they fit (the routing launch of the
  // same call returns at once then): a GEMM1 on device-read tokens only
  if (route_small_in_kernel && (!g.sw.enabled || g.route_in_kernel || rows_on_device == nullptr ||
                                g.num_experts > kFusedMaxExperts))
    return hipErrorInvalidValue;
  GemmArgs eight = g;
  if (route_small_in_kernel) eight.route_in_kernel = 2;
  if (wide && rows_on_device != nullptr) {
    // the bound selects WIDE, but the rows are known on the device only: both kernels go out,
    // and the one the routed rows do not select returns at once (the 8-wave one without the
    // WIDE GEMM2's direct writes, which the requant then leaves switched off)
    GemmArgs d = g;
    d.dual_rows = rows_on_device;
    d.dual_min_rows = dual_min_rows > 0 ? dual_min_rows : gemm_wide_min_rows(g.num_experts);
    // (a smaller threshold than the default only where the 8-wave kernel never routes itself)
    if (d.dual_min_rows <= kFusedMaxTasks && route_small_in_kernel) return hipErrorInvalidValue;
    eight.dual_rows = d.dual_rows;
    eight.dual_min_rows = d.dual_min_rows;
    eight.row_dest = nullptr;
    eight.y_direct = nullptr;
    eight.direct_flag = nullptr;
    const hipError_t err = g.sw.enabled ? launch_engines<true, true>(eight, max_rows, num_cus, stream)
                                        : launch_engines<false, false>(eight, max_rows, num_cus, stream);
    if (err != hipSuccess) return err;
    return g.sw.enabled ? launch_wide<true, true, kWideBM1>(d, max_rows, num_cus, stream)
                        : launch_wide<false, false, kWideBM2>(d, max_rows, num_cus, stream);
  }
  if (wide && route_small_in_kernel) return hipErrorInvalidValue;  // (rows_on_device is set)
  if (g.sw.enabled)
    return wide ? launch_wide<true, true, kWideBM1>(g, max_rows, num_cus, stream)
                : launch_engines<true, true>(eight, max_rows, num_cus, stream);
  return wide ? launch_wide<false, false, kWideBM2>(g, max_rows, num_cus, stream)
              : launch_engines<false, false>(eight, max_rows, num_cus, stream);
}

}  // namespace mmoe
