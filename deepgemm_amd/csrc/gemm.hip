// gemm.hip -- grouped FP8 (OCP e4m3) GEMM on gfx950 MFMA for the expert-contiguous rows.
//
//   c[r, n] = bf16( (sum_k a[r,k] * b[e,n,k]) * a_scale[r] * b_scale[e,n] ),  e = expert of r
//
// GEMM1 (gate+up, N = 2I, K = H) gathers its A rows straight from the token matrix through
// row_token (the dispatch "pull" of the reference, K1: megamoe/dcu_megamoe_large_opt/K1_fused/
// k1_fused_ext.cu:479-746), so no grouped copy of x is materialised. GEMM2 (N = H, K = I)
// reads the requantised SwiGLU rows. B is the Marlin nt_kpack2 weight
// (deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66): per 16-row tile, each 16-byte
// k-block of the 16 rows is 256 contiguous bytes, so a BN x BK weight tile is BN/16 runs of
// BK*16 contiguous bytes -- fully coalesced, and copied to LDS without reshuffling.
//
// LDS layout of a stage (both operands): 16-row x 16-byte blocks, block (rb, kb) at
// (rb*BK/16 + kb)*256, row ri of the block at +ri*16. A 32x32x64 MFMA operand for lane l
// (row l%32, k-half l/32) is two 16-byte reads of consecutive blocks; 16 consecutive lanes read
// 256 contiguous bytes, so the reads are bank-conflict free. The k order inside an MFMA step is
// the same permutation for A and B, hence irrelevant to the dot product.
//
// Work distribution: persistent workgroups stride over (m-tile, n-tile) pairs; the m-tiles of
// every expert are enumerated on device from counts[], so the host never synchronises.
#include "common.cuh"
#include "kernels.h"

namespace mmoe {

namespace {

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int kThreads = WM * WN * kWave;
  static constexpr int kKB = BK / 16;
  static constexpr int kAChunks = BM * BK / 16;
  static constexpr int kBChunks = BN * BK / 16;
  static constexpr int kAPerThread = kAChunks / kThreads;
  static constexpr int kBPerThread = kBChunks / kThreads;
  static constexpr int kWTM = BM / WM, kWTN = BN / WN;
  static constexpr int kTM = kWTM / 32, kTN = kWTN / 32;
  static constexpr int kStageBytes = (BM + BN) * BK;
  static constexpr int kSmemBytes = 2 * kStageBytes;
  static_assert(kAChunks % kThreads == 0 && kBChunks % kThreads == 0, "stage not divisible");
  static_assert(kWTM % 32 == 0 && kWTN % 32 == 0, "wave tile must be 32-aligned");
  static_assert(BK % 64 == 0, "BK must be a multiple of the MFMA k (64)");
};

using DecodeCfg = GemmCfg<32, 128, 128, 1, 4>;
using PrefillCfg = GemmCfg<128, 128, 128, 2, 2>;

__device__ __forceinline__ v8i make_v8i(const int4& lo, const int4& hi) {
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

template <class Cfg, bool kGather>
__global__ __launch_bounds__(Cfg::kThreads) void grouped_gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_prefix[kMaxExperts + 1];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int wm = wave / Cfg::WN;
  const int wn = wave % Cfg::WN;
  const int E = g.num_experts;

  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      s_prefix[e] = acc;
      acc += (g.counts[e] + Cfg::BM - 1) / Cfg::BM;
    }
    s_prefix[E] = acc;
  }
  __syncthreads();
  const int n_tiles = g.n / Cfg::BN;
  const int total = s_prefix[E] * n_tiles;
  const int k_steps = g.k / Cfg::BK;
  const int64_t b_rowtile_stride = static_cast<int64_t>(g.k) * 16;  // bytes per 16-row tile

  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    const int mt_global = t / n_tiles;
    const int nt = t - mt_global * n_tiles;
    // expert: last e with s_prefix[e] <= mt_global
    int lo = 0, hi = E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_prefix[mid] <= mt_global) lo = mid; else hi = mid;
    }
    const int e = lo;
    const int mt = mt_global - s_prefix[e];
    const int row0 = g.offsets[e] + mt * Cfg::BM;
    const int mrows = min(Cfg::BM, g.counts[e] - mt * Cfg::BM);
    const int n0 = nt * Cfg::BN;

    const uint8_t* a_src[Cfg::kAPerThread];
#pragma unroll
    for (int i = 0; i < Cfg::kAPerThread; ++i) {
      const int c = tid + i * Cfg::kThreads;
      const int rb = c / (16 * Cfg::kKB);
      const int rem = c - rb * 16 * Cfg::kKB;
      const int kb = rem >> 4;
      const int r = rb * 16 + (rem & 15);
      if (r < mrows) {
        const int row = row0 + r;
        const int64_t src_row = kGather ? static_cast<int64_t>(g.row_token[row]) : row;
        a_src[i] = g.a + src_row * g.lda + kb * 16;
      } else {
        a_src[i] = nullptr;
      }
    }
    const uint8_t* b_src[Cfg::kBPerThread];
#pragma unroll
    for (int i = 0; i < Cfg::kBPerThread; ++i) {
      const int c = tid + i * Cfg::kThreads;
      const int rb = c / (16 * Cfg::kKB);
      const int rem = c - rb * 16 * Cfg::kKB;
      b_src[i] = g.b + (static_cast<int64_t>(e) * (g.n / 16) + n0 / 16 + rb) * b_rowtile_stride + rem * 16;
    }

    int4 ra[Cfg::kAPerThread];
    int4 rbv[Cfg::kBPerThread];
    auto load_stage = [&](int k0) {
#pragma unroll
      for (int i = 0; i < Cfg::kAPerThread; ++i)
        ra[i] = a_src[i] != nullptr ? *reinterpret_cast<const int4*>(a_src[i] + k0) : make_int4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < Cfg::kBPerThread; ++i)
        rbv[i] = *reinterpret_cast<const int4*>(b_src[i] + static_cast<int64_t>(k0) * 16);
    };
    auto store_stage = [&](int buf) {
      uint8_t* sa = smem + buf * Cfg::kStageBytes;
      uint8_t* sb = sa + Cfg::BM * Cfg::BK;
#pragma unroll
      for (int i = 0; i < Cfg::kAPerThread; ++i)
        *reinterpret_cast<int4*>(sa + (tid + i * Cfg::kThreads) * 16) = ra[i];
#pragma unroll
      for (int i = 0; i < Cfg::kBPerThread; ++i)
        *reinterpret_cast<int4*>(sb + (tid + i * Cfg::kThreads) * 16) = rbv[i];
    };

    v16f acc[Cfg::kTM][Cfg::kTN];
#pragma unroll
    for (int i = 0; i < Cfg::kTM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::kTN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    auto compute_stage = [&](int buf) {
      const uint8_t* sa = smem + buf * Cfg::kStageBytes;
      const uint8_t* sb = sa + Cfg::BM * Cfg::BK;
#pragma unroll
      for (int ks = 0; ks < Cfg::BK / 64; ++ks) {
        const int kb = ks * 4 + (lane >> 5) * 2;
        v8i av[Cfg::kTM];
        v8i bv[Cfg::kTN];
#pragma unroll
        for (int tm = 0; tm < Cfg::kTM; ++tm) {
          const int r = wm * Cfg::kWTM + tm * 32 + (lane & 31);
          const int off = ((r >> 4) * Cfg::kKB + kb) * 256 + (r & 15) * 16;
          av[tm] = make_v8i(*reinterpret_cast<const int4*>(sa + off),
                            *reinterpret_cast<const int4*>(sa + off + 256));
        }
#pragma unroll
        for (int tn = 0; tn < Cfg::kTN; ++tn) {
          const int cidx = wn * Cfg::kWTN + tn * 32 + (lane & 31);
          const int off = ((cidx >> 4) * Cfg::kKB + kb) * 256 + (cidx & 15) * 16;
          bv[tn] = make_v8i(*reinterpret_cast<const int4*>(sb + off),
                            *reinterpret_cast<const int4*>(sb + off + 256));
        }
#pragma unroll
        for (int tm = 0; tm < Cfg::kTM; ++tm)
#pragma unroll
          for (int tn = 0; tn < Cfg::kTN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                av[tm], bv[tn], acc[tm][tn], 0, 0, 0, 0, 0, 0);
      }
    };

    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < k_steps; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < k_steps) load_stage((kt + 1) * Cfg::BK);
      compute_stage(cur);
      if (kt + 1 < k_steps) store_stage(cur ^ 1);
      __syncthreads();
    }

    // epilogue: scale and round to bf16. MFMA 32x32 result: lane l, register v holds
    // row 8*(v/4) + 4*(l/32) + v%4, column l%32.
    const float* bs = g.b_scale + static_cast<int64_t>(e) * g.n + n0;
#pragma unroll
    for (int tm = 0; tm < Cfg::kTM; ++tm) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * Cfg::kWTM + tm * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (r < mrows) {
          const int row = row0 + r;
          const float sa = kGather ? g.a_scale[g.row_token[row]] : g.a_scale[row];
          uint16_t* crow = g.c + static_cast<int64_t>(row) * g.n + n0;
#pragma unroll
          for (int tn = 0; tn < Cfg::kTN; ++tn) {
            const int col = wn * Cfg::kWTN + tn * 32 + (lane & 31);
            crow[col] = f32_to_bf16(acc[tm][tn][v] * sa * bs[col]);
          }
        }
      }
    }
  }
}

template <class Cfg>
hipError_t launch_cfg(const GemmArgs& g, int max_rows, int num_cus, int per_cu,
                      hipStream_t stream) {
  const int64_t max_mtiles = (static_cast<int64_t>(max_rows) + Cfg::BM - 1) / Cfg::BM + g.num_experts;
  const int64_t max_tiles = max_mtiles * (g.n / Cfg::BN);
  int64_t grid = static_cast<int64_t>(num_cus) * per_cu;
  if (grid > max_tiles) grid = max_tiles;
  if (grid < 1) grid = 1;
  if (g.row_token != nullptr) {
    hipLaunchKernelGGL((grouped_gemm_kernel<Cfg, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(Cfg::kThreads), Cfg::kSmemBytes, stream, g);
  } else {
    hipLaunchKernelGGL((grouped_gemm_kernel<Cfg, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(Cfg::kThreads), Cfg::kSmemBytes, stream, g);
  }
  return hipGetLastError();
}

}  // namespace

bool gemm_shape_supported(int n, int k) {
  return n > 0 && k > 0 && n % 128 == 0 && k % 128 == 0;
}

hipError_t launch_grouped_gemm(const GemmArgs& g, GemmShape shape, int max_rows, int num_cus,
                               hipStream_t stream) {
  if (max_rows <= 0) return hipSuccess;
  if (shape == GemmShape::kDecode) return launch_cfg<DecodeCfg>(g, max_rows, num_cus, 4, stream);
  return launch_cfg<PrefillCfg>(g, max_rows, num_cus, 2, stream);
}

}  // namespace mmoe
