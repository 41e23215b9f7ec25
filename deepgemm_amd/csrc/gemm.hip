// gemm.hip -- grouped FP8 (OCP e4m3) GEMM on gfx950 MFMA for the expert-contiguous rows.
//
//   c[r, n] = bf16( (sum_k a[r,k] * b[e,n,k]) * a_scale[r] * b_scale[e,n] ),  e = expert of r
//
// GEMM1 (gate+up, N = 2I, K = H) gathers its A rows straight from the token matrix through
// row_token (the dispatch "pull" of the reference, K1: megamoe/dcu_megamoe_large_opt/K1_fused/
// k1_fused_ext.cu:479-746), so no grouped copy of x is materialised. GEMM2 (N = H, K = I)
// reads the requantised SwiGLU rows. B is the Marlin nt_kpack2 weight
// (deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66): per 16-row tile, each 16-byte
// k-block of the 16 rows is 256 contiguous bytes.
//
// One persistent kernel, two tile engines chosen per expert on the device from counts[]:
//
//  * STREAM engine (experts with <= 64 rows: decode). The layer is HBM-bound on the weights, so
//    a tile is (expert, 64 output columns, all <= 64 rows) and its four waves split K four ways.
//    Every wave loads its MFMA operands straight from global memory into registers (Marlin
//    gives each lane 16 contiguous k-bytes of one weight row; 16 lanes read 256 contiguous
//    bytes) through a 2-4 deep register ring, so 12-24 KB per wave is in flight with no LDS
//    and no barrier in the K loop. The four K-partials are summed through LDS in a fixed order.
//  * TILE engine (larger experts: prefill). 128x128 output tiles, BK = 128, A and B staged
//    through double-buffered LDS in 16-row x 16-byte blocks (block (rb, kb) at
//    (rb*BK/16 + kb)*256); a 32x32x64 MFMA operand of lane l (row l%32, k-half l/32) is two
//    16-byte reads of consecutive blocks, 16 lanes reading 256 contiguous bytes (conflict-free).
//
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
// register ring depth (64-k steps in flight per wave): 4 with one 32-row subtile, 2 with two
template <int MT>
struct StreamDepth { static constexpr int value = MT == 1 ? 4 : 2; };
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

template <bool kGather>
__device__ __forceinline__ float row_scale(const GemmArgs& g, int row) {
  return kGather ? g.a_scale[g.row_token[row]] : g.a_scale[row];
}

template <bool kGather>
__device__ __forceinline__ const uint8_t* a_row_ptr(const GemmArgs& g, int row) {
  const int64_t src = kGather ? static_cast<int64_t>(g.row_token[row]) : row;
  return g.a + src * g.lda;
}

// ------------------------------------------------------------------ STREAM engine
template <bool kGather, int MT>
__device__ void stream_tile(const GemmArgs& g, int e, int row0, int mrows, int n0, uint8_t* smem) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int ksteps = g.k / 64;
  const int s_begin = wave * ksteps / kGemmWaves;
  const int nsteps = (wave + 1) * ksteps / kGemmWaves - s_begin;
  const int khalf = (lane >> 5) * 32;

  const uint8_t* ap[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 32 + (lane & 31);
    ap[mt] = a_row_ptr<kGather>(g, row0 + (r < mrows ? r : 0)) + khalf + s_begin * 64;
  }
  const uint8_t* bp[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = n0 + ct * 32 + (lane & 31);
    bp[ct] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + (n >> 4)) * (static_cast<int64_t>(g.k) * 16) +
             (n & 15) * 16 + (lane >> 5) * 512 + static_cast<int64_t>(s_begin) * 1024;
  }

  constexpr int kStreamDepth = StreamDepth<MT>::value;
  int4 ar[kStreamDepth][MT][2];
  int4 br[kStreamDepth][2][2];
  auto issue = [&](int slot, int s) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ar[slot][mt][0] = ld16(ap[mt] + s * 64);
      ar[slot][mt][1] = ld16(ap[mt] + s * 64 + 16);
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      br[slot][ct][0] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024);
      br[slot][ct][1] = ld16(bp[ct] + static_cast<int64_t>(s) * 1024 + 256);
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
  if (nsteps >= kStreamDepth && nsteps % kStreamDepth == 0) {
    // Straight-line ring: every load is unconditional, so the compiler's wait counts stay
    // exact (each step waits only for its own slot, the oldest loads in flight).
    // The scheduling barriers keep the issue order slot by slot, so a slot's loads are always
    // the oldest in flight when it is consumed (wait = vmcnt of the younger slots).
#pragma unroll
    for (int d = 0; d < kStreamDepth; ++d) {
      issue(d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int i = 0; i + kStreamDepth < nsteps; i += kStreamDepth) {
#pragma unroll
      for (int d = 0; d < kStreamDepth; ++d) {
        compute(d);
        issue(d, i + d + kStreamDepth);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < kStreamDepth; ++d) compute(d);
  } else {
    // short or uneven K slices (small shapes): one step at a time
    for (int s = 0; s < nsteps; ++s) {
      issue(0, s);
      compute(0);
    }
  }

  // fixed-order reduction of the four K partials: red[wave][mt][ct][v][lane]
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        red[(((wave * 2 + mt) * 2 + ct) * 16 + v) * kWave + lane] = acc[mt][ct][v];
  __syncthreads();
  const int pmt = wave >> 1, pct = wave & 1;  // (mt, ct) pair this wave finishes
  if (pmt < MT) {
    const float bs = g.b_scale[static_cast<int64_t>(e) * g.n + n0 + pct * 32 + (lane & 31)];
    uint16_t* cbase = g.c + n0 + pct * 32 + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kGemmWaves; ++w) s += red[(((w * 2 + pmt) * 2 + pct) * 16 + v) * kWave + lane];
      const int r = pmt * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      if (r < mrows) {
        const int row = row0 + r;
        cbase[static_cast<int64_t>(row) * g.n] = f32_to_bf16(s * row_scale<kGather>(g, row) * bs);
      }
    }
  }
}

// ------------------------------------------------------------------ TILE engine
template <bool kGather>
__device__ void tile_tile(const GemmArgs& g, int e, int row0, int mrows, int n0, uint8_t* smem) {
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
    b_src[i] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + n0 / 16 + rb) * (static_cast<int64_t>(g.k) * 16) + rem * 16;
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
        const int cidx = wn * WTN + tn * 32 + (lane & 31);
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

  const float* bs = g.b_scale + static_cast<int64_t>(e) * g.n + n0;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = wm * WTM + tm * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      if (r < mrows) {
        const int row = row0 + r;
        const float sa = row_scale<kGather>(g, row);
        uint16_t* crow = g.c + static_cast<int64_t>(row) * g.n + n0;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const int col = wn * WTN + tn * 32 + (lane & 31);
          crow[col] = f32_to_bf16(acc[tm][tn][v] * sa * bs[col]);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ persistent dispatcher
template <bool kGather>
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
      tile_tile<kGather>(g, e, g.offsets[e] + mt * kTileBM, min(kTileBM, cnt - mt * kTileBM),
                         nb * kTileBN, smem);
    } else {
      const int nt = g.n / kStreamBN;
      const int mt = local / nt;
      const int nb = local - mt * nt;
      const int mrows = min(kStreamMaxRows, cnt - mt * kStreamMaxRows);
      if (mrows > 32)
        stream_tile<kGather, 2>(g, e, g.offsets[e] + mt * kStreamMaxRows, mrows, nb * kStreamBN, smem);
      else
        stream_tile<kGather, 1>(g, e, g.offsets[e] + mt * kStreamMaxRows, mrows, nb * kStreamBN, smem);
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
  if (g.row_token != nullptr) {
    hipLaunchKernelGGL(grouped_gemm_kernel<true>, dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
  } else {
    hipLaunchKernelGGL(grouped_gemm_kernel<false>, dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), kSmemBytes, stream, g);
  }
  return hipGetLastError();
}

}  // namespace mmoe
