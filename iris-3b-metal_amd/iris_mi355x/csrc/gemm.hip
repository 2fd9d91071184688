// BF16 GEMM on gfx950 MFMA: C[m, n] = sum_k A[m, k] * B[n, k] (+ bias[n]), FP32 accumulate.
//
// Both operands are K-contiguous ("NT"), the natural layout of nn.Linear weights, so every
// MFMA operand fragment is one 16-byte LDS read. A 256-thread workgroup computes a BM x BN
// tile with four waves in a 2 x 2 arrangement; each wave owns a (BM/2) x (BN/2) block built
// from v_mfma_f32_32x32x16_bf16. The weight fragment is the MFMA's A operand and the
// activation fragment its B operand, so each lane ends up holding four consecutive output
// columns of one row: the epilogue stores 8 (BF16) or 16 (FP32) contiguous bytes per lane.
//
// Pipeline: the K loop is double-buffered in LDS (rows padded to 144 bytes so the 16-lane
// phases of ds_read_b128 hit 64 distinct banks); the next K tile is fetched into registers
// while the current one feeds the MFMAs, then written to the other buffer; one barrier per
// K tile. Workgroup ids are remapped so consecutive tiles (which share the weight tile)
// run on the same XCD and hit its L2.
#include "iris_common.hpp"

namespace iris {
namespace {

constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // elements per LDS row: 144 bytes

struct GemmGroup {
  const bf16* a;
  const bf16* b;
  const float* bias;
  void* c;
  int m;
  int tiles_m;
  int tile_begin;
};

struct GemmArgs {
  GemmGroup g0, g1;
  int ngroups;
  int n, k;
  long lda, ldb, ldc;
  int total_tiles;
};

template <typename TC>
__device__ __forceinline__ void store_out4(TC* p, float v0, float v1, float v2, float v3) {
  store4(p, f32x4{v0, v1, v2, v3});
}

template <int BM, int BN, int EPI, typename TC>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int A_CHUNKS = BM * kBK / 8 / 256;
  constexpr int B_CHUNKS = BN * kBK / 8 / 256;
  constexpr int STAGE = (BM + BN) * kLdsStride;
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * STAGE];

  int tile = xcd_remap(blockIdx.x, p.total_tiles);
  const bool second = p.ngroups > 1 && tile >= p.g1.tile_begin;
  const bf16* __restrict__ A = second ? p.g1.a : p.g0.a;
  const bf16* __restrict__ B = second ? p.g1.b : p.g0.b;
  const float* __restrict__ bias = second ? p.g1.bias : p.g0.bias;
  TC* __restrict__ C = static_cast<TC*>(second ? p.g1.c : p.g0.c);
  const int M = second ? p.g1.m : p.g0.m;
  const int tiles_m = second ? p.g1.tiles_m : p.g0.tiles_m;
  tile -= second ? p.g1.tile_begin : 0;
  const int tn = tile / tiles_m;
  const int tm = tile - tn * tiles_m;
  const int N = p.n;
  const long lda = p.lda, ldb = p.ldb;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;

  // global -> register fetch addresses: chunk idx = tid + 256 i -> row idx / 8, column chunk idx % 8
  const int ld_row = tid >> 3;
  const int ld_col = (tid & 7) * 8;
  // 32-bit element offsets (the host checks m * lda and n * ldb stay below 2^31)
  int a_off[A_CHUNKS], b_off[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i)
    a_off[i] = min(tm * BM + ld_row + 32 * i, M - 1) * static_cast<int>(lda) + ld_col;
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i)
    b_off[i] = min(tn * BN + ld_row + 32 * i, N - 1) * static_cast<int>(ldb) + ld_col;

  bf16x8 ra[A_CHUNKS], rb[B_CHUNKS];
  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

  const int KT = p.k / kBK;
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) ra[i] = *reinterpret_cast<const bf16x8*>(A + a_off[i] + kt * kBK);
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) rb[i] = *reinterpret_cast<const bf16x8*>(B + b_off[i] + kt * kBK);
  };
  auto stash = [&](int buf) {
    bf16* As = lds + buf * STAGE;
    bf16* Bs = As + BM * kLdsStride;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i)
      *reinterpret_cast<bf16x8*>(As + (ld_row + 32 * i) * kLdsStride + ld_col) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i)
      *reinterpret_cast<bf16x8*>(Bs + (ld_row + 32 * i) * kLdsStride + ld_col) = rb[i];
  };

  fetch(0);
  stash(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) fetch(kt + 1);
    const bf16* As = lds + cur * STAGE + (wm * WM + l32) * kLdsStride + g * 8;
    const bf16* Bs = lds + cur * STAGE + BM * kLdsStride + (wn * WN + l32) * kLdsStride + g * 8;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 wf[FN], xf[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) wf[i] = *reinterpret_cast<const bf16x8*>(Bs + i * 32 * kLdsStride + ks * 16);
#pragma unroll
      for (int j = 0; j < FM; ++j) xf[j] = *reinterpret_cast<const bf16x8*>(As + j * 32 * kLdsStride + ks * 16);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) stash(cur ^ 1);
    __syncthreads();
  }

  // epilogue: acc[i][j][r] = C[m, n] with n = tile + 8 (r / 4) + 4 g + r % 4, m = tile + l32
  const long ldc = p.ldc;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = tm * BM + wm * WM + j * 32 + l32;
    if (m >= M) continue;
    TC* crow = C + static_cast<long>(m) * ldc;
    if constexpr (EPI == IRIS_EPI_SILU_MUL) {
#pragma unroll
      for (int i = 0; i < FN; i += 2) {
        const int nbase = tn * BN + wn * WN + i * 32;
        if (nbase >= N) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = silu(acc[i][j][4 * q + e]) * acc[i + 1][j][4 * q + e];
          store_out4(crow + nbase / 2 + 8 * q + 4 * g, v[0], v[1], v[2], v[3]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < FN; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n0 = tn * BN + wn * WN + i * 32 + 8 * q + 4 * g;
          if (n0 >= N) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
          if (bias) {
            const f32x4 bv = load4(bias + n0);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += bv[e];
          }
          store_out4(crow + n0, v[0], v[1], v[2], v[3]);
        }
      }
    }
  }
}

template <int BM, int BN>
int launch_tile(GemmArgs& args, int c_dtype, int epilogue, hipStream_t stream) {
  const dim3 grid(args.total_tiles);
  if (epilogue == IRIS_EPI_SILU_MUL) {
    if (c_dtype == IRIS_BF16)
      gemm_kernel<BM, BN, IRIS_EPI_SILU_MUL, bf16><<<grid, 256, 0, stream>>>(args);
    else
      gemm_kernel<BM, BN, IRIS_EPI_SILU_MUL, float><<<grid, 256, 0, stream>>>(args);
  } else {
    if (c_dtype == IRIS_BF16)
      gemm_kernel<BM, BN, IRIS_EPI_NONE, bf16><<<grid, 256, 0, stream>>>(args);
    else
      gemm_kernel<BM, BN, IRIS_EPI_NONE, float><<<grid, 256, 0, stream>>>(args);
  }
  return check_launch("gemm_bf16");
}

// Tile shape: the largest tile that still gives about one full round of workgroups on the
// 256 CUs; smaller tiles trade MFMA intensity for occupancy on the N = 1280 / 2560 shapes.
int pick_tile(long m_total, int n, int forced) {
  if (forced >= 0) return forced;
  const long t256 = ((m_total + 255) / 256) * ((n + 255) / 256);
  if (t256 >= 224) return 0;
  const long t256x128 = ((m_total + 255) / 256) * ((n + 127) / 128);
  if (t256x128 >= 224) return 1;
  return 2;
}

int g_forced_tile = -1;

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_gemm_bf16_grouped(int groups, const void* const* a, const void* const* b,
                                      const float* const* bias, void* const* c, const int* m, int c_dtype, int n,
                                      int k, long lda, long ldb, long ldc, int epilogue, hipStream_t stream) {
  IRIS_REQUIRE(groups == 1 || groups == 2, "gemm: 1 or 2 groups");
  IRIS_REQUIRE(c_dtype == IRIS_F32 || c_dtype == IRIS_BF16, "gemm: unknown output dtype");
  IRIS_REQUIRE(epilogue == IRIS_EPI_NONE || epilogue == IRIS_EPI_SILU_MUL, "gemm: unknown epilogue");
  IRIS_REQUIRE(n > 0 && k > 0 && k % kBK == 0, "gemm: need n > 0 and k %% 64 == 0 (got n=%d k=%d)", n, k);
  IRIS_REQUIRE(n % 4 == 0, "gemm: n %% 4 == 0 required (got %d)", n);
  IRIS_REQUIRE(epilogue != IRIS_EPI_SILU_MUL || n % 64 == 0, "gemm: the SwiGLU epilogue needs n %% 64 == 0");
  IRIS_REQUIRE(lda >= k && ldb >= k && lda % 8 == 0 && ldb % 8 == 0, "gemm: lda/ldb must be >= k and multiples of 8");
  IRIS_REQUIRE(ldc >= (epilogue == IRIS_EPI_SILU_MUL ? n / 2 : n) && ldc % 4 == 0, "gemm: bad ldc");
  GemmArgs args{};
  args.ngroups = groups;
  args.n = n;
  args.k = k;
  args.lda = lda;
  args.ldb = ldb;
  args.ldc = ldc;
  long m_total = 0;
  for (int i = 0; i < groups; ++i) {
    IRIS_REQUIRE(m[i] >= 0, "gemm: negative m");
    IRIS_REQUIRE(m[i] == 0 || (a[i] && b[i] && c[i]), "gemm: null pointer");
    IRIS_REQUIRE(!a[i] || (aligned(a[i], 16) && aligned(b[i], 16) && aligned(c[i], 16)),
                 "gemm: operands must be 16-byte aligned");
    IRIS_REQUIRE(!bias || !bias[i] || epilogue == IRIS_EPI_NONE, "gemm: bias is not supported with SwiGLU");
    m_total += m[i];
  }
  IRIS_REQUIRE(static_cast<long>(n) * ldb < (1L << 31), "gemm: weight too large for 32-bit offsets");
  for (int i = 0; i < groups; ++i)
    IRIS_REQUIRE(static_cast<long>(m[i]) * lda < (1L << 31), "gemm: activation too large for 32-bit offsets");
  const int tile = pick_tile(m_total, n, g_forced_tile);
  const int bm = tile == 2 ? 128 : 256;
  const int bn = tile == 0 ? 256 : 128;
  const int tiles_n = (n + bn - 1) / bn;
  int begin = 0;
  GemmGroup* gs[2] = {&args.g0, &args.g1};
  for (int i = 0; i < groups; ++i) {
    GemmGroup& gg = *gs[i];
    gg.a = static_cast<const bf16*>(a[i]);
    gg.b = static_cast<const bf16*>(b[i]);
    gg.bias = bias ? bias[i] : nullptr;
    gg.c = c[i];
    gg.m = m[i];
    gg.tiles_m = (m[i] + bm - 1) / bm;
    gg.tile_begin = begin;
    begin += gg.tiles_m * tiles_n;
  }
  if (groups == 1) args.g1 = args.g0, args.g1.tile_begin = begin;
  args.total_tiles = begin;
  if (begin == 0) return IRIS_OK;
  switch (tile) {
    case 0:
      return launch_tile<256, 256>(args, c_dtype, epilogue, stream);
    case 1:
      return launch_tile<256, 128>(args, c_dtype, epilogue, stream);
    default:
      return launch_tile<128, 128>(args, c_dtype, epilogue, stream);
  }
}

extern "C" int iris_gemm_bf16(const void* a, const void* b, const float* bias, void* c, int c_dtype, int m, int n,
                              int k, long lda, long ldb, long ldc, int epilogue, hipStream_t stream) {
  const void* as[1] = {a};
  const void* bs[1] = {b};
  const float* biases[1] = {bias};
  void* cs[1] = {c};
  int ms[1] = {m};
  return iris_gemm_bf16_grouped(1, as, bs, biases, cs, ms, c_dtype, n, k, lda, ldb, ldc, epilogue, stream);
}

// Tuning hook: force a tile shape (0: 256x256, 1: 256x128, 2: 128x128, -1: automatic).
extern "C" int iris_gemm_force_tile(int tile) {
  IRIS_REQUIRE(tile >= -1 && tile <= 2, "gemm_force_tile: tile in -1..2");
  g_forced_tile = tile;
  return IRIS_OK;
}
