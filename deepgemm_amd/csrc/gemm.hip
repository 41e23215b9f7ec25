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
// Two persistent kernels per GEMM (two tile engines); each expert's engine is chosen on the
// device from its routed row count and each kernel skips the other engine's experts:
//  * STREAM engine (<= 64 rows: decode, HBM-bound on the weights). One wave per tile =
//    (expert, 64 output columns, all <= 64 rows) over the full K; the wave loads its MFMA
//    operands straight from global memory into registers (Marlin gives each lane 16 contiguous
//    k-bytes of one weight row; 16 lanes read 256 contiguous bytes) through a straight-line
//    register ring 4 steps deep, with no LDS and no barrier. With ~2 waves per SIMD there are
//    about as many resident waves as decode tiles, so a wave streams one long tile.
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

constexpr int kGemmThreads = 256;  // TILE engine workgroup
constexpr int kMaxGemmExperts = 256;
constexpr int kStreamMaxRows = 64;  // experts up to this many rows use the STREAM engine
constexpr int kStreamBN = 64;
constexpr int kStreamDepth = 4;     // register ring depth (64-k steps in flight), one subtile
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
// One wave computes a whole tile: (expert, 64 output columns, MT 32-row subtiles) over the full
// K, so there is no cross-wave reduction and no barrier. Its MFMA operands come straight from
// global memory into a register ring kStreamDepth steps deep: every load is unconditional and
// the scheduling barriers keep the issue order slot by slot, so the compiler's wait for a slot
// leaves the younger slots in flight. The k order of the accumulation is the same as the TILE
// engine's (sequential 64-k steps), so both engines produce the same bits.
template <bool kGather, bool kSwiglu, int MT>
__device__ void stream_wave_tile(const GemmArgs& g, int e, int row0, int mrows, int nb) {
  constexpr int kDepth = MT == 1 ? kStreamDepth : kStreamDepth - 1;
  const int lane = lane_id();
  const int nsteps = g.k / 64;

  const uint8_t* ap[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 32 + (lane & 31);
    ap[mt] = a_row_ptr<kGather>(g, row0 + (r < mrows ? r : 0)) + (lane >> 5) * 32;
  }
  const uint8_t* bp[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = weight_row<kSwiglu>(g, nb, kStreamBN, ct * 32 + (lane & 31));
    bp[ct] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
             (n & 15) * 16 + (lane >> 5) * 512;
  }

  int4 ar[kDepth][MT][2];
  int4 br[kDepth][2][2];
  auto issue = [&](int slot, int s) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      br[slot][ct][0] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024);
      br[slot][ct][1] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024 + 256);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ar[slot][mt][0] = ld16(ap[mt] + s * 64);
      ar[slot][mt][1] = ld16(ap[mt] + s * 64 + 16);
    }
  };
  v16f acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][ct][v] = 0.0f;
  auto compute = [&](int slot) {
    const v8i b0 = make_v8i(br[slot][0][0], br[slot][0][1]);
    const v8i b1 = make_v8i(br[slot][1][0], br[slot][1][1]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const v8i a = make_v8i(ar[slot][mt][0], ar[slot][mt][1]);
      acc[mt][0] = mfma_fp8(a, b0, acc[mt][0]);
      acc[mt][1] = mfma_fp8(a, b1, acc[mt][1]);
    }
  };
  if (nsteps >= kDepth && nsteps % kDepth == 0) {
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
    for (int s = 0; s < nsteps; ++s) {  // short K (small shapes): one step at a time
      issue(0, s);
      compute(0);
    }
  }

  if (!kSwiglu) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int col = nb * kStreamBN + ct * 32 + (lane & 31);
      const float bs = g.b_scale[static_cast<int64_t>(e) * g.n + col];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = mt * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
          if (r < mrows) {
            const int row = row0 + r;
            g.c[static_cast<int64_t>(row) * g.n + col] =
                f32_to_bf16(acc[mt][ct][v] * row_scale<kGather>(g, row) * bs);
          }
        }
    }
  } else {
    const int chan = nb * (kStreamBN / 2) + (lane & 31);
    const float wsg = g.b_scale[static_cast<int64_t>(e) * g.n + chan];
    const float wsu = g.b_scale[static_cast<int64_t>(e) * g.n + g.sw.inter + chan];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = mt * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        const bool ok = r < mrows;
        const int row = row0 + (ok ? r : 0);
        float yv = 0.0f;
        if (ok) {
          yv = swiglu_value(g, acc[mt][0][v], acc[mt][1][v], row_scale<kGather>(g, row), wsg, wsu,
                            g.sw.row_weight[row]);
          g.sw.y[static_cast<int64_t>(row) * g.sw.inter + chan] = yv;
        }
        const float m = half_wave_max(fabsf(yv));
        if (ok && (lane & 31) == 0) atomicMax(g.sw.amax + row, __float_as_uint(m));
      }
  }
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

// ------------------------------------------------------------------ persistent dispatchers
// Wave 0 of the workgroup fills s_prefix[0..E] with the exclusive prefix of the tiles of the
// experts this kernel owns (`tile_kernel`: experts on the TILE engine, else STREAM).
__device__ void enumerate_tiles(const GemmArgs& g, bool tile_kernel, int* s_prefix) {
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
        if (tile == tile_kernel)
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
}

__device__ __forceinline__ int expert_of_tile(const int* s_prefix, int E, int t) {
  int lo = 0, hi = E;  // last e with s_prefix[e] <= t
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_prefix[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

template <bool kGather, bool kSwiglu>
__global__ __launch_bounds__(kWave, 2) void stream_gemm_kernel(GemmArgs g) {
  __shared__ int s_prefix[kMaxGemmExperts + 1];
  enumerate_tiles(g, false, s_prefix);
  __syncthreads();
  const int E = g.num_experts;
  const int total = s_prefix[E];
  const int nt = g.n / kStreamBN;
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    const int e = expert_of_tile(s_prefix, E, t);
    const int local = t - s_prefix[e];
    const int mt = local / nt;
    const int nb = local - mt * nt;
    const int row0 = g.offsets[e] + mt * kStreamMaxRows;
    const int mrows = min(kStreamMaxRows, g.counts[e] - mt * kStreamMaxRows);
    if (mrows > 32)
      stream_wave_tile<kGather, kSwiglu, 2>(g, e, row0, mrows, nb);
    else
      stream_wave_tile<kGather, kSwiglu, 1>(g, e, row0, mrows, nb);
  }
}

template <bool kGather, bool kSwiglu>
__global__ __launch_bounds__(kGemmThreads, 2) void tile_gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_prefix[kMaxGemmExperts + 1];
  enumerate_tiles(g, true, s_prefix);
  __syncthreads();
  const int E = g.num_experts;
  const int total = s_prefix[E];
  const int nt = g.n / kTileBN;
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    const int e = expert_of_tile(s_prefix, E, t);
    const int local = t - s_prefix[e];
    const int mt = local / nt;
    const int nb = local - mt * nt;
    tile_tile<kGather, kSwiglu>(g, e, g.offsets[e] + mt * kTileBM,
                                min(kTileBM, g.counts[e] - mt * kTileBM), nb, smem);
    __syncthreads();
  }
}

template <bool kGather, bool kSwiglu>
hipError_t launch_engines(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  if (g.engine != GemmEngine::kTile) {
    const int64_t tiles =
        (static_cast<int64_t>(max_rows) / kStreamMaxRows + g.num_experts) * (g.n / kStreamBN);
    int64_t grid = static_cast<int64_t>(num_cus) * 8;  // 2 waves per SIMD
    if (grid > tiles) grid = tiles;
    hipLaunchKernelGGL((stream_gemm_kernel<kGather, kSwiglu>), dim3(static_cast<unsigned>(grid)),
                       dim3(kWave), 0, stream, g);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (g.engine != GemmEngine::kStream) {
    const int64_t tiles =
        (static_cast<int64_t>(max_rows) / kTileBM + g.num_experts) * (g.n / kTileBN);
    int64_t grid = static_cast<int64_t>(num_cus) * 2;
    if (grid > tiles) grid = tiles;
    hipLaunchKernelGGL((tile_gemm_kernel<kGather, kSwiglu>), dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace

bool gemm_shape_supported(int n, int k) {
  return n > 0 && k > 0 && n % 128 == 0 && k % 128 == 0;
}

hipError_t launch_grouped_gemm(const GemmArgs& g, int max_rows, int num_cus, hipStream_t stream) {
  if (max_rows <= 0) return hipSuccess;
  if (g.num_experts > kMaxGemmExperts) return hipErrorInvalidValue;
  if (g.sw.enabled) {
    if (g.row_token == nullptr || g.n != 2 * g.sw.inter) return hipErrorInvalidValue;
    return launch_engines<true, true>(g, max_rows, num_cus, stream);
  }
  if (g.row_token != nullptr) return hipErrorInvalidValue;
  return launch_engines<false, false>(g, max_rows, num_cus, stream);
}

}  // namespace mmoe
