// gemm.hip -- grouped FP8 (OCP e4m3) GEMMs of the layer on gfx950 MFMA, over the
// expert-contiguous routed rows.
//
// GEMM1 (gate+up, K = H) gathers its A rows straight from the token matrix through row_token
// (the dispatch "pull" of the reference's K1, megamoe/dcu_megamoe_large_opt/K1_fused/
// k1_fused_ext.cu:479-746), so no grouped copy of x exists, and fuses the K2 stage
// (megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:254-377) into its epilogue:
//   h = bf16(acc * x_sf[token] * w1_sf[e, n])       for the gate and the up column of a channel
//   y = silu(min(h_g, c)) * clamp(h_u, -c, c) * w    (fp32, left to right)
//   amax[row] = max |y| over the row (atomic max of the float bits: order-free, deterministic)
// Each output tile holds matching gate and up channels, so SwiGLU is elementwise in registers.
// The per-row requant (a = max(amax, 1e-4); act = e4m3(clip(y * 448/a)); act_scale = a/448)
// runs as its own small kernel: a cross-workgroup hand-off inside GEMM1 would need an
// agent-scope release per tile, which on gfx950 writes back the whole (per-XCD, non-coherent)
// L2 -- measured 4x slower than the kernel boundary.
// GEMM2 (down, K = I) reads act/act_scale and writes the bf16 partial rows for the combine:
//   part[r, n] = bf16((sum_k act[r,k] * w2[e,n,k]) * act_scale[r] * w2_sf[e,n]).
//
// B is the Marlin nt_kpack2 weight (deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66):
// per 16-row tile, each 16-byte k-block of the 16 rows is 256 contiguous bytes.
//
// One persistent kernel per GEMM, two tile engines chosen per expert on the device from its
// routed row count:
//  * STREAM engine (<= 64 rows: decode, HBM-bound on the weights). Tile = (expert, 64 output
//    columns, all rows). The four waves split K; each wave loads its MFMA operands straight from
//    global memory into registers (Marlin gives each lane 16 contiguous k-bytes of one weight
//    row; 16 lanes read 256 contiguous bytes) through a straight-line register ring 4 steps
//    deep, with no LDS and no barrier in the K loop, one 32-row subtile at a time. The
//    K-partials are summed through LDS in a fixed order.
//  * TILE engine (more rows: prefill, MFMA-bound). 128x128 output tiles, BK = 128, A and B
//    staged through double-buffered LDS in 16-row x 16-byte blocks (block (rb, kb) at
//    (rb*BK/16 + kb)*256); a 32x32x64 MFMA operand of lane l (row l%32, k-half l/32) is two
//    16-byte reads of consecutive blocks, 16 lanes reading 256 contiguous bytes (conflict-free).
// In both engines lane l supplies k-bytes [32*(l/32), 32*(l/32)+32) of each 64-k MFMA step for
// A and B alike; any such bijection gives the same dot product.
#include "common.cuh"
#include "kernels.h"

namespace mmoe {

namespace {

constexpr int kGemmThreads = 256;
constexpr int kGemmWaves = kGemmThreads / kWave;
constexpr int kMaxGemmExperts = 256;
constexpr int kStreamMaxRows = 64;  // experts up to this many rows use the STREAM engine
constexpr int kStreamBN = 64;
constexpr int kStreamDepth = 4;     // register ring depth: 64-k steps in flight per wave
constexpr int kTileBM = 128, kTileBN = 128, kTileBK = 128;
constexpr int kTileWM = 2, kTileWN = 2;
constexpr int kSmemBytes = 65536;

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

__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <bool kGather>
__device__ __forceinline__ float row_scale(const GemmArgs& g, int row) {
  return kGather ? g.a_scale[g.row_token[row]] : g.a_scale[row];
}

template <bool kGather>
__device__ __forceinline__ const uint8_t* a_row_ptr(const GemmArgs& g, int row) {
  const int64_t src = kGather ? static_cast<int64_t>(g.row_token[row]) : row;
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
  float gh = bf16_round(gacc * xs * wsg);
  float uh = bf16_round(uacc * xs * wsu);
  if (g.sw.has_clamp) {
    uh = fminf(g.sw.clamp, fmaxf(-g.sw.clamp, uh));
    gh = fminf(g.sw.clamp, gh);
  }
  return gh * (1.0f / (1.0f + expf(-gh))) * uh * route_w;
}

// max over the 32 lanes of each half-wave (the 32 channels of one output row)
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ------------------------------------------------------------------ STREAM engine
// One 32-row subtile of a STREAM tile: the full K pass, the K-partial reduction and the epilogue.
template <bool kGather, bool kSwiglu>
__device__ void stream_subtile(const GemmArgs& g, int e, int row0, int mrows, int nb, uint8_t* smem) {
  constexpr int kDepth = kStreamDepth;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int ksteps = g.k / 64;
  const int s_begin = wave * ksteps / kGemmWaves;
  const int nsteps = (wave + 1) * ksteps / kGemmWaves - s_begin;

  const int r_lane = lane & 31;
  const uint8_t* ap = a_row_ptr<kGather>(g, row0 + (r_lane < mrows ? r_lane : 0)) +
                      (lane >> 5) * 32 + s_begin * 64;
  const uint8_t* bp[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = weight_row<kSwiglu>(g, nb, kStreamBN, ct * 32 + (lane & 31));
    bp[ct] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
             (n & 15) * 16 + (lane >> 5) * 512 + static_cast<int64_t>(s_begin) * 1024;
  }

  int4 ar[kDepth][2];
  int4 br[kDepth][2][2];
  auto issue = [&](int slot, int s) {
    ar[slot][0] = ld16(ap + s * 64);
    ar[slot][1] = ld16(ap + s * 64 + 16);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      br[slot][ct][0] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024);
      br[slot][ct][1] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024 + 256);
    }
  };
  v16f acc[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[ct][v] = 0.0f;
  auto compute = [&](int slot) {
    const v8i a = make_v8i(ar[slot][0], ar[slot][1]);
    acc[0] = mfma_fp8(a, make_v8i(br[slot][0][0], br[slot][0][1]), acc[0]);
    acc[1] = mfma_fp8(a, make_v8i(br[slot][1][0], br[slot][1][1]), acc[1]);
  };
  if (nsteps >= kDepth && nsteps % kDepth == 0) {
    // Straight-line ring: every load is unconditional and the scheduling barriers keep the
    // issue order slot by slot, so a slot's loads are the oldest in flight when it is consumed
    // (the compiler's wait = vmcnt of the younger slots).
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      issue(d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int i = 0; i + kDepth < nsteps; i += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        compute(d);
        issue(d, i + d + kDepth);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) compute(d);
  } else {
    // short or uneven K slices (small shapes): one step at a time
    for (int s = 0; s < nsteps; ++s) {
      issue(0, s);
      compute(0);
    }
  }

  // fixed-order reduction of the four K partials: red[wave][ct][v][lane]
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int v = 0; v < 16; ++v) red[((wave * 2 + ct) * 16 + v) * kWave + lane] = acc[ct][v];
  __syncthreads();
  auto partial_sum = [&](int ct, int v) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kGemmWaves; ++w) s += red[((w * 2 + ct) * 16 + v) * kWave + lane];
    return s;
  };
  // wave w finishes registers v in [4w, 4w+4) (rows 8*w + 4*(lane/32) + 0..3) of both columns
  if (!kSwiglu) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int col = nb * kStreamBN + ct * 32 + (lane & 31);
      const float bs = g.b_scale[static_cast<int64_t>(e) * g.n + col];
#pragma unroll
      for (int vv = 0; vv < 4; ++vv) {
        const int v = wave * 4 + vv;
        const float s = partial_sum(ct, v);
        const int r = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (r < mrows) {
          const int row = row0 + r;
          g.c[static_cast<int64_t>(row) * g.n + col] = f32_to_bf16(s * row_scale<kGather>(g, row) * bs);
        }
      }
    }
  } else {
    const int chan = nb * (kStreamBN / 2) + (lane & 31);
    const float wsg = g.b_scale[static_cast<int64_t>(e) * g.n + chan];
    const float wsu = g.b_scale[static_cast<int64_t>(e) * g.n + g.sw.inter + chan];
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
      const int v = wave * 4 + vv;
      const float ga = partial_sum(0, v);
      const float ua = partial_sum(1, v);
      const int r = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      float yv = 0.0f;
      const bool ok = r < mrows;
      const int row = row0 + (ok ? r : 0);
      if (ok) {
        yv = swiglu_value(g, ga, ua, row_scale<kGather>(g, row), wsg, wsu, g.sw.row_weight[row]);
        g.sw.y[static_cast<int64_t>(row) * g.sw.inter + chan] = yv;
      }
      const float m = half_wave_max(fabsf(yv));
      if (ok && (lane & 31) == 0) atomicMax(g.sw.amax + row, __float_as_uint(m));
    }
  }
  __syncthreads();  // the reduction buffer is reused by the next subtile / tile
}

// A STREAM tile: (expert, 64 columns, <= 64 rows) as one or two 32-row subtiles; the second
// subtile re-reads the same weight slice, which the first left in L2.
template <bool kGather, bool kSwiglu>
__device__ void stream_tile(const GemmArgs& g, int e, int row0, int mrows, int nb, uint8_t* smem) {
  for (int sub = 0; sub * 32 < mrows; ++sub)
    stream_subtile<kGather, kSwiglu>(g, e, row0 + sub * 32, min(32, mrows - sub * 32), nb, smem);
}

// ------------------------------------------------------------------ TILE engine
template <bool kGather, bool kSwiglu>
__device__ void tile_tile(const GemmArgs& g, int e, int row0, int mrows, int nb, uint8_t* smem) {
  constexpr int BM = kTileBM, BN = kTileBN, BK = kTileBK;
  constexpr int KB = BK / 16;
  constexpr int kAPer = BM * BK / 16 / kGemmThreads;
  constexpr int kBPer = BN * BK / 16 / kGemmThreads;
  constexpr int kStage = (BM + BN) * BK;
  constexpr int WTM = BM / kTileWM, WTN = BN / kTileWN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int wm = wave / kTileWN, wn = wave % kTileWN;
  const int k_steps = g.k / BK;

  const uint8_t* a_src[kAPer];
#pragma unroll
  for (int i = 0; i < kAPer; ++i) {
    const int c = tid + i * kGemmThreads;
    const int rb = c / (16 * KB);
    const int rem = c - rb * 16 * KB;
    const int r = rb * 16 + (rem & 15);
    a_src[i] = r < mrows ? a_row_ptr<kGather>(g, row0 + r) + (rem >> 4) * 16 : nullptr;
  }
  const uint8_t* b_src[kBPer];
#pragma unroll
  for (int i = 0; i < kBPer; ++i) {
    const int c = tid + i * kGemmThreads;
    const int rb = c / (16 * KB);
    const int rem = c - rb * 16 * KB;
    const int n = weight_row<kSwiglu>(g, nb, BN, rb * 16);  // row-tile aligned
    b_src[i] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) + rem * 16;
  }
  int4 ra[kAPer];
  int4 rbv[kBPer];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kAPer; ++i) ra[i] = a_src[i] != nullptr ? ld16(a_src[i] + k0) : make_int4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kBPer; ++i) rbv[i] = ld16(b_src[i] + static_cast<int64_t>(k0) * 16);
  };
  auto store_stage = [&](int buf) {
    uint8_t* sa = smem + buf * kStage;
    uint8_t* sb = sa + BM * BK;
#pragma unroll
    for (int i = 0; i < kAPer; ++i) *reinterpret_cast<int4*>(sa + (tid + i * kGemmThreads) * 16) = ra[i];
#pragma unroll
    for (int i = 0; i < kBPer; ++i) *reinterpret_cast<int4*>(sb + (tid + i * kGemmThreads) * 16) = rbv[i];
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // B tile column of the wave's column tile tn: without SwiGLU wn*64 + tn*32; with SwiGLU the
  // wave's gate columns (tn = 0) sit at wn*32 and the matching up columns (tn = 1) at 64+wn*32.
  auto b_col = [&](int tn) { return kSwiglu ? tn * (BN / 2) + wn * 32 : wn * WTN + tn * 32; };

  auto compute_stage = [&](int buf) {
    const uint8_t* sa = smem + buf * kStage;
    const uint8_t* sb = sa + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      const int kb = ks * 4 + (lane >> 5) * 2;
      v8i av[TM], bv[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const int r = wm * WTM + tm * 32 + (lane & 31);
        const int off = ((r >> 4) * KB + kb) * 256 + (r & 15) * 16;
        av[tm] = make_v8i(*reinterpret_cast<const int4*>(sa + off), *reinterpret_cast<const int4*>(sa + off + 256));
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int cidx = b_col(tn) + (lane & 31);
        const int off = ((cidx >> 4) * KB + kb) * 256 + (cidx & 15) * 16;
        bv[tn] = make_v8i(*reinterpret_cast<const int4*>(sb + off), *reinterpret_cast<const int4*>(sb + off + 256));
      }
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = mfma_fp8(av[tm], bv[tn], acc[tm][tn]);
    }
  };

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int kt = 0; kt < k_steps; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < k_steps) load_stage((kt + 1) * BK);
    compute_stage(cur);
    if (kt + 1 < k_steps) store_stage(cur ^ 1);
    __syncthreads();
  }

  if (!kSwiglu) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * WTM + tm * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (r < mrows) {
          const int row = row0 + r;
          const float sa = row_scale<kGather>(g, row);
          uint16_t* crow = g.c + static_cast<int64_t>(row) * g.n;
#pragma unroll
          for (int tn = 0; tn < TN; ++tn) {
            const int col = nb * BN + b_col(tn) + (lane & 31);
            crow[col] = f32_to_bf16(acc[tm][tn][v] * sa * g.b_scale[static_cast<int64_t>(e) * g.n + col]);
          }
        }
      }
    }
  } else {
    static_assert(TN == 2, "SwiGLU epilogue pairs one gate and one up column tile");
    const int chan = nb * (BN / 2) + wn * 32 + (lane & 31);
    const float wsg = g.b_scale[static_cast<int64_t>(e) * g.n + chan];
    const float wsu = g.b_scale[static_cast<int64_t>(e) * g.n + g.sw.inter + chan];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * WTM + tm * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        const bool ok = r < mrows;
        const int row = row0 + (ok ? r : 0);
        float yv = 0.0f;
        if (ok) {
          yv = swiglu_value(g, acc[tm][0][v], acc[tm][1][v], row_scale<kGather>(g, row), wsg, wsu,
                            g.sw.row_weight[row]);
          g.sw.y[static_cast<int64_t>(row) * g.sw.inter + chan] = yv;
        }
        const float m = half_wave_max(fabsf(yv));
        if (ok && (lane & 31) == 0) atomicMax(g.sw.amax + row, __float_as_uint(m));
      }
    }
  }
}

// ------------------------------------------------------------------ persistent dispatcher
template <bool kGather, bool kSwiglu>
__global__ __launch_bounds__(kGemmThreads, 2) void grouped_gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_prefix[kMaxGemmExperts + 1];
  __shared__ unsigned char s_tile_engine[kMaxGemmExperts];
  const int E = g.num_experts;
  const int lane = lane_id();
  if (threadIdx.x < kWave) {
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int e = e0 + lane;
      int tiles = 0;
      if (e < E) {
        const int cnt = g.counts[e];
        const bool tile = g.engine == GemmEngine::kTile ||
                          (g.engine == GemmEngine::kAuto && cnt > kStreamMaxRows);
        s_tile_engine[e] = tile ? 1 : 0;
        tiles = tile ? (cnt + kTileBM - 1) / kTileBM * (g.n / kTileBN)
                     : (cnt + kStreamMaxRows - 1) / kStreamMaxRows * (g.n / kStreamBN);
      }
      int inc = tiles;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int u = __shfl_up(inc, off, kWave);
        if (lane >= off) inc += u;
      }
      if (e < E) s_prefix[e] = carry + inc - tiles;
      carry += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) s_prefix[E] = carry;
  }
  __syncthreads();
  const int total = s_prefix[E];
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    int lo = 0, hi = E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_prefix[mid] <= t) lo = mid; else hi = mid;
    }
    const int e = lo;
    const int local = t - s_prefix[e];
    const int cnt = g.counts[e];
    if (s_tile_engine[e]) {
      const int nt = g.n / kTileBN;
      const int mt = local / nt;
      const int nb = local - mt * nt;
      tile_tile<kGather, kSwiglu>(g, e, g.offsets[e] + mt * kTileBM,
                                  min(kTileBM, cnt - mt * kTileBM), nb, smem);
    } else {
      const int nt = g.n / kStreamBN;
      const int mt = local / nt;
      const int nb = local - mt * nt;
      stream_tile<kGather, kSwiglu>(g, e, g.offsets[e] + mt * kStreamMaxRows,
                                    min(kStreamMaxRows, cnt - mt * kStreamMaxRows), nb, smem);
    }
    __syncthreads();
  }
}

}  // namespace

bool gemm_shape_supported(int n, int k) {
  return n > 0 && k > 0 && n % 128 == 0 && k % 128 == 0;
}

hipError_t launch_grouped_gemm(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  if (max_rows <= 0) return hipSuccess;
  if (g.num_experts > kMaxGemmExperts) return hipErrorInvalidValue;
  // upper bound of the tiles of either engine, for the persistent grid size
  const int64_t stream_tiles =
      (static_cast<int64_t>(max_rows) / kStreamMaxRows + g.num_experts) * (g.n / kStreamBN);
  int64_t grid = static_cast<int64_t>(num_cus) * 2;
  if (grid > stream_tiles) grid = stream_tiles;
  if (grid < 1) grid = 1;
  if (g.sw.enabled) {
    if (g.row_token == nullptr || g.n != 2 * g.sw.inter) return hipErrorInvalidValue;
    hipLaunchKernelGGL((grouped_gemm_kernel<true, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
  } else {
    if (g.row_token != nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL((grouped_gemm_kernel<false, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
  }
  return hipGetLastError();
}

}  // namespace mmoe
