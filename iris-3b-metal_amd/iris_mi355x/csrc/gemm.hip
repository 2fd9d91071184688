// BF16 GEMM on gfx950 MFMA: C[m, n] = sum_k A[m, k] * B[n, k] (+ bias[n]), FP32 accumulate.
//
// Both operands are K-contiguous ("NT"), the natural layout of nn.Linear weights, so every
// MFMA operand fragment is one 16-byte LDS read. The weight fragment is the MFMA's A operand
// and the activation fragment its B operand, so each lane ends up holding four consecutive
// output columns of one row. LDS tiles are XOR-swizzled so the fragment reads are bank-conflict
// free, and workgroup ids are remapped so that the tiles running concurrently on one XCD form
// an 8 x 4 block and share their operands through that XCD's L2.
//
// Three kernels:
// - gemm_w4h_kernel (the default for plain, bias and SwiGLU outputs and the q|k|v store): four
//   waves, one per SIMD, in a 2 x 2 grid of v_mfma_f32_16x16x32_bf16 blocks; K tiles staged
//   through registers (16-byte buffer loads two K tiles ahead) into a 2-stage LDS ring;
//   288 x 160, 256 x 160, 128 x 160, 256 x 256 and 192 x 256 tiles. gemm_w4h_pair_kernel runs
//   two of its GEMMs in one grid (SwiGLU's two column parts; the q|k|v store and the gate
//   columns beside it), which saves the boundary between two launches.
// - gemm_w4_kernel: the same design on v_mfma_f32_32x32x16_bf16 (256 x 256, 192 x 256),
//   forced-only (a tuning and test reference).
// - gemm_kernel: eight waves, K tiles global -> LDS with buffer_load_dwordx4 ... lds into a ring
//   of STAGES buffers (no register staging; a 32-bit VGPR byte offset per load, the K position
//   in an SGPR, the LDS target wave-uniform), v_mfma_f32_32x32x16_bf16; the SiLU epilogue's
//   kernel (the four-wave kernels have none).
// The MFMA shape of a launch follows from its epilogue alone (mfma16_family), so a row's
// result never depends on the row count or the tile chosen.
#include "iris_common.hpp"

#include <type_traits>

namespace iris {
namespace {

constexpr int kBK = 64;

struct GemmGroup {
  const bf16* a;
  const bf16* b;
  const float* bias;
  void* c;
  int m;
  int tiles_m;
  int tile_begin;
};

// The q | k | v projection's store with the attention inputs' per-head RMSNorm + RoPE
// (kEpiQkRope): output columns [0, 128 heads) are the Q heads, the next 128 kv_heads the K heads,
// written normed and rotated to q [B, heads, n_dst, 128] and k [B, kv_heads, n_dst, 128] at
// position dst_offset + token (row m of group g is token m % rows_per_batch[g] of batch item
// m / rows_per_batch[g]); the columns after them (the V heads) go to C unchanged.
struct QkRope {
  bf16 *q, *k;
  const float *cos, *sin;  // [positions, 64]
  const float *q_weight0, *q_weight1, *k_weight0, *k_weight1;  // per group, 128 gains each
  int rows_per_batch0, rows_per_batch1, dst_offset0, dst_offset1;
  int n_dst, heads, kv_heads;
  float eps;
  // with vt: the V heads go transposed to vt [B, kv_heads, 128, n_vt] (the layout of
  // v_heads_t) instead of to C; needs every group's rows_per_batch % 256 == 0 and
  // dst_offset % 16 == 0, so that a tile's 256 rows are whole 16-position groups of one item
  bf16* vt;
  int n_vt;
};

constexpr int kEpiQkRope = 3;  // internal epilogue code, next to the public IRIS_EPI_* values

struct GemmArgs {
  GemmGroup g0, g1;
  int ngroups;
  int n, k;
  long lda, ldb, ldc;
  int total_tiles;
  QkRope qk;  // kEpiQkRope only
};

template <typename TC>
__device__ __forceinline__ void store_out4(TC* p, float v0, float v1, float v2, float v3) {
  store4(p, f32x4{v0, v1, v2, v3});
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Same, and also all LDS reads of this wave (lgkmcnt = 0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// LDS layout: each operand tile is BM (or BN) rows of BK bf16, unpadded; the 16-byte chunk c
// of row r is stored at chunk c ^ swz(r) so that the 16 rows read by one ds_read_b128 phase
// cover all 64 banks. Tiles are filled by buffer_load_dwordx4 ... lds, which writes lane i's
// 16 bytes at LDS base + 16 i: each lane therefore fetches the global chunk that belongs
// at its LDS position.
template <int BK>
__device__ __forceinline__ int swz(int r) {
  constexpr int CPR = BK / 8;
  return (r / (16 / CPR)) % CPR;
}

// One workgroup's output tile: the logical tile id (XCD remap) picks the group, then groups
// of 8 row tiles sweep all column tiles, so that the ~32 tiles running at once on one XCD form
// an 8 x 4 block and share their operands through that XCD's L2.
struct TileJob {
  const bf16* a;
  const bf16* b;
  const float* bias;
  void* c;
  int m, tm, tn;
  int group;
};

template <int BM, int BN>
__device__ __forceinline__ TileJob locate_tile_at(const GemmArgs& p, int tile) {
  const bool second = p.ngroups > 1 && tile >= p.g1.tile_begin;
  const GemmGroup& gr = second ? p.g1 : p.g0;
  tile -= second ? p.g1.tile_begin : 0;
  const int tiles_n = (p.n + BN - 1) / BN;
  constexpr int GM = 8;
  const int group = tile / (GM * tiles_n);
  const int gm = min(GM, gr.tiles_m - group * GM);
  const int in_group = tile - group * GM * tiles_n;
  return TileJob{gr.a, gr.b, gr.bias, gr.c, gr.m, group * GM + in_group % gm, in_group / gm, second ? 1 : 0};
}

template <int BM, int BN>
__device__ __forceinline__ TileJob locate_tile(const GemmArgs& p) {
  return locate_tile_at<BM, BN>(p, xcd_remap(blockIdx.x, p.total_tiles));
}

// Persistent workgroups: round r of G workgroups (wg = 0 .. G - 1) covers logical tiles r G ..
// r G + G - 1, remapped per XCD as a one-round launch would be; -1 when this workgroup has no
// tile in round r (only in the last one). Workgroup wg must run on XCD wg % 8.
__device__ __forceinline__ int persistent_tile(const GemmArgs& p, int round, int wg, int G) {
  const int base = round * G;
  const int count = min(G, p.total_tiles - base);
  return wg < count ? base + xcd_remap(wg, count) : -1;
}
__device__ __forceinline__ int persistent_tile(const GemmArgs& p, int round) {
  return persistent_tile(p, round, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
}

// kEpiQkRope, while the accumulators are staged: the Q and K gains of this tile's group go to
// LDS (qk_gain, 256 floats) and thread r's rotary table row (tile row r) to registers.
template <int BM>
__device__ __forceinline__ void qk_tables(const TileJob& job, const QkRope& qk, float* qk_gain, f32x4 (&qk_cos)[16],
                                          f32x4 (&qk_sin)[16]) {
  const int tid = threadIdx.x;
  const int M = job.m, tm = job.tm;
  const float* __restrict__ gains = tid < 32 ? (job.group ? qk.q_weight1 : qk.q_weight0)
                                             : (job.group ? qk.k_weight1 : qk.k_weight0);
  if (tid < 64) store4(qk_gain + 4 * tid, load4(gains + 4 * (tid & 31)));
  const int rpb = job.group ? qk.rows_per_batch1 : qk.rows_per_batch0;
  const int mm = min(tm * BM + tid, M - 1);  // (rows past M read a valid row, unused)
  const int b = mm / rpb;
  const long pos = (job.group ? qk.dst_offset1 : qk.dst_offset0) + (mm - b * rpb);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    qk_cos[i] = load4(qk.cos + pos * 64 + 4 * i);
    qk_sin[i] = load4(qk.sin + pos * 64 + 4 * i);
  }
}

// kEpiQkRope, once the BF16 tile is staged in LDS (256 outputs per row, 4-element unit u of row
// r at u ^ 2 (r & 15)): thread r normalises and rotates the Q / K heads of tile row r in place
// (two 128-column heads per row, 16 chunks each), then the tile leaves in 16-byte row chunks:
// Q / K rows to q / k at their token's position, the V columns to C (or transposed to vt).
template <int BM, int NW>
__device__ __forceinline__ void qk_store(bf16* cl, const TileJob& job, int N, long ldc, const QkRope& qk,
                                         const float* qk_gain, const f32x4 (&qk_cos)[16], const f32x4 (&qk_sin)[16]) {
  constexpr int OUT_N = 256, MASK = 15, CHUNKS = 32;
  const int tid = threadIdx.x;
  const int M = job.m, tm = job.tm, tn = job.tn;
  bf16* __restrict__ C = static_cast<bf16*>(job.c);
  const int n_out = N;
  const int col0 = tn * OUT_N;
  const int nq = qk.heads * 128, nqk = nq + qk.kv_heads * 128;
  const int rpb = job.group ? qk.rows_per_batch1 : qk.rows_per_batch0;
  const int dst_offset = job.group ? qk.dst_offset1 : qk.dst_offset0;
  if (tm * BM + tid < M) {
    bf16* row = cl + tid * OUT_N;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int n0 = col0 + 128 * hh;  // (the same for the whole workgroup)
      if (n0 >= n_out || n0 >= nqk) continue;
      const float* gain = qk_gain + (n0 < nq ? 0 : 128);
      auto chunk = [&](int c) { return reinterpret_cast<bf16x8*>(row + 8 * ((16 * hh + c) ^ (tid & MASK))); };
      float ss[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const bf16x8 v = *chunk(c);
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = to_f32(v[e]);
        ss[c] = head_chunk_sq(a);
      }
      const float rs = head_rms_scale(head_sum_tree(ss), qk.eps);
#pragma unroll
      for (int c = 0; c < 16; ++c) {  // (read again: keeping the head in registers spills)
        const bf16x8 v = *chunk(c);
        float a[8], w[8], y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = to_f32(v[e]);
        load8(gain + 8 * c, w);
        head_scale_rope(a, rs, w, qk_cos[c], qk_sin[c], y);
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = from_f32<bf16>(y[e]);
        *chunk(c) = o;
      }
    }
  }
  __syncthreads();
  if (qk.vt) {
    // V heads transposed: thread t gathers dim t % 128 for positions 8 c .. 8 c + 7 of the
    // tile's tokens (each 16-position group in the slot order of vt_slot), c = t / 128 + 2 j;
    // a wave's lanes read 64 consecutive dims of one tile row (no LDS bank conflicts) and
    // store 16 bytes each into 64 rows of vt
    const int b = (tm * BM) / rpb;
    const long p0 = dst_offset + (tm * BM - b * rpb);  // a multiple of 16
    const int d = tid & 127;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int n0 = col0 + 128 * hh;  // (the same for the whole workgroup)
      if (n0 < nqk || n0 >= n_out) continue;
      const int vh = (n0 - nqk) >> 7;
      const int col = 128 * hh + d;
      bf16* vtd = qk.vt + ((static_cast<long>(b) * qk.kv_heads + vh) * 128 + d) * static_cast<long>(qk.n_vt) + p0;
#pragma unroll 4
      for (int j = 0; j < 16; ++j) {
        const int c8 = (tid >> 7) + 2 * j;  // (wave-uniform)
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = vt_slot(8 * c8 + e);  // tile row holding this position's token
          o[e] = cl[i * OUT_N + 4 * ((col >> 2) ^ (2 * (i & MASK))) + (col & 3)];
        }
        *reinterpret_cast<bf16x8*>(vtd + 8 * c8) = o;
      }
    }
  }
#pragma unroll 4
  for (int idx = tid; idx < BM * CHUNKS; idx += 64 * NW) {
    const int r = idx / CHUNKS;
    const int c = idx - r * CHUNKS;
    const int m = tm * BM + r;
    const int n0 = col0 + 8 * c;
    if (m >= M || n0 >= n_out) continue;
    if (n0 >= nqk && qk.vt) continue;  // (written transposed above)
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(cl + r * OUT_N + 8 * (c ^ (r & MASK)));
    if (n0 >= nqk) {  // V heads
      *reinterpret_cast<bf16x8*>(C + static_cast<long>(m) * ldc + n0) = v;
      continue;
    }
    const bool is_q = n0 < nq;
    const int head = (is_q ? n0 : n0 - nq) >> 7;
    const int b = m / rpb;
    const long pos = dst_offset + (m - b * rpb);
    bf16* dst = is_q ? qk.q + ((static_cast<long>(b) * qk.heads + head) * qk.n_dst + pos) * 128
                     : qk.k + ((static_cast<long>(b) * qk.kv_heads + head) * qk.n_dst + pos) * 128;
    *reinterpret_cast<bf16x8*>(dst + 8 * (c & 15)) = v;
  }
}

// Epilogue shared by the kernels: acc[i][j][r] = C[m, n] with n = tile + wave col + 32 i +
// 8 (r / 4) + 4 g + r % 4, m = tile + wave row + 32 j + l32; BF16 output through the LDS ring.
// `mid` runs once the accumulators are no longer needed (after they are staged in LDS, or at
// the end for FP32 output); the persistent kernel issues its next loads there.
template <int BM, int BN, int WM, int WN, int FM, int FN, int NW, int RING, int EPI, typename TC, typename Mid>
__device__ __forceinline__ void store_tile(f32x16 (&acc)[FN][FM], bf16* lds, const TileJob& job, int N, long ldc,
                                           int wm, int wn, const QkRope& qk, Mid&& mid) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int M = job.m, tm = job.tm, tn = job.tn;
  const float* __restrict__ bias = job.bias;
  TC* __restrict__ C = static_cast<TC*>(job.c);
  if constexpr (sizeof(TC) == 2) {
    // BF16 output: stage the tile through LDS (the K ring is free once every wave is past its
    // last MFMA) so that each store instruction writes whole 512-byte row segments instead of
    // 16-byte pieces of 32 rows. 4-element unit u of row r sits at unit u ^ 2 (r & MASK).
    constexpr int OUT_N = EPI == IRIS_EPI_SILU_MUL ? BN / 2 : BN;
    constexpr int UNITS = OUT_N / 4;
    // the XOR must stay inside the row: within 32-unit blocks when the row holds whole ones,
    // else within 16-unit blocks (rows of 48 units for BN = 192)
    constexpr int MASK = UNITS % 32 == 0 ? 15 : (UNITS % 16 == 0 ? 7 : 0);
    static_assert(UNITS % 16 == 0 || UNITS < 16, "output tile width");
    static_assert(BM * OUT_N <= RING, "output tile must fit in the LDS ring");
    bf16* cl = lds;
    __syncthreads();
    // kEpiQkRope: the Q and K gains of this tile's group go to LDS, and thread r's rotary table row
    // (tile row r) to registers, while the accumulators are staged
    __shared__ float qk_gain[EPI == kEpiQkRope ? 256 : 1];
    [[maybe_unused]] f32x4 qk_cos[EPI == kEpiQkRope ? 16 : 1], qk_sin[EPI == kEpiQkRope ? 16 : 1];
    if constexpr (EPI == kEpiQkRope) {
      static_assert(BM == 64 * NW, "one tile row per thread");
      qk_tables<BM>(job, qk, qk_gain, qk_cos, qk_sin);
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int r = wm * WM + j * 32 + l32;
      bf16* crow_l = cl + r * OUT_N;
      const int sw = 2 * (r & MASK);
      if constexpr (EPI == IRIS_EPI_SILU_MUL) {
#pragma unroll
        for (int i = 0; i < FN; i += 2) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = silu(acc[i][j][4 * q + e]) * acc[i + 1][j][4 * q + e];
            const int u = ((wn * WN + i * 32) / 2 + 8 * q + 4 * g) / 4;
            store_out4(crow_l + 4 * (u ^ sw), v[0], v[1], v[2], v[3]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < FN; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int nl = wn * WN + i * 32 + 8 * q + 4 * g;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
            if (bias) {
              const f32x4 bv = load4(bias + min(tn * BN + nl, N - 4));
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] += bv[e];
            }
            if constexpr (EPI == IRIS_EPI_SILU)
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = silu(v[e]);
            store_out4(crow_l + 4 * ((nl / 4) ^ sw), v[0], v[1], v[2], v[3]);
          }
        }
      }
    }
    __syncthreads();
    mid();
    constexpr int CHUNKS = OUT_N / 8;  // 16-byte chunks per row
    const int n_out = EPI == IRIS_EPI_SILU_MUL ? N / 2 : N;
    const int col0 = tn * OUT_N;
    if constexpr (EPI == kEpiQkRope) {
      static_assert(OUT_N == 256 && MASK == 15 && CHUNKS == 32, "two heads of 16 chunks per row");
      qk_store<BM, NW>(cl, job, N, ldc, qk, qk_gain, qk_cos, qk_sin);
      return;
    }
#pragma unroll 4
    for (int idx = tid; idx < BM * CHUNKS; idx += 64 * NW) {
      const int r = idx / CHUNKS;
      const int c = idx - r * CHUNKS;
      const int m = tm * BM + r;
      const int n0 = col0 + 8 * c;
      if (m >= M || n0 >= n_out) continue;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(cl + r * OUT_N + 8 * (c ^ (r & MASK)));
      TC* dst = C + static_cast<long>(m) * ldc + n0;
      if (n0 + 8 <= n_out) {
        *reinterpret_cast<bf16x8*>(dst) = v;
      } else {
        *reinterpret_cast<bf16x4*>(dst) = bf16x4{v[0], v[1], v[2], v[3]};  // n_out % 4 == 0
      }
    }
    return;
  }
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
          if constexpr (EPI == IRIS_EPI_SILU)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = silu(v[e]);
          store_out4(crow + n0, v[0], v[1], v[2], v[3]);
        }
      }
    }
  }
  mid();
}

// Loads of part `part` when a K tile's lpw loads are dealt round-robin into `parts` parts.
constexpr int part_loads(int lpw, int parts, int part) { return part < parts ? (lpw - part + parts - 1) / parts : 0; }

// Instruction order inside one k-step: one MFMA (its operands were read a whole k-step
// earlier), then every fragment read of the next k-step (NR), then this k-step's global loads,
// then the remaining MFMAs (NM in all), so each read has all but one MFMA of the k-step to
// land. Without these hints the scheduler sinks the reads below the MFMAs that free their
// registers and waits for them at the start of the next k-step with nothing left in flight.
template <int NR, int NM, int LOADS>
__device__ __forceinline__ void order_kstep() {
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // MFMA
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);                           // DS read
  if constexpr (LOADS > 0) __builtin_amdgcn_sched_group_barrier(0x010, LOADS, 0);  // VMEM
  __builtin_amdgcn_sched_group_barrier(0x008, NM - 1, 0);                       // MFMA
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int PARTS, int EPI, typename TC>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_kernel(GemmArgs p) {
  constexpr int NW = WGM * WGN;             // waves per workgroup
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int KS = BK / 16;               // MFMA k-steps per K tile
  constexpr int CPR = BK / 8;               // 16-byte chunks per row
  constexpr int RPL = 64 / CPR;             // rows per wave-wide 1 KB load
  constexpr int A_LOADS = BM / RPL / NW;    // load instructions per wave per stage
  constexpr int B_LOADS = BN / RPL / NW;
  constexpr int LPW = A_LOADS + B_LOADS;
  constexpr int A_STAGE = BM * BK, STAGE = (BM + BN) * BK;
  static_assert(A_LOADS * RPL * NW == BM && B_LOADS * RPL * NW == BN, "tile / wave split");
  static_assert(STAGES >= 2 && (STAGES - 2) * LPW < 64, "pipeline depth");
  static_assert(PARTS >= 1 && PARTS <= 4 && PARTS <= KS && PARTS <= LPW, "load parts");
  __shared__ __attribute__((aligned(1024))) bf16 lds[STAGES * STAGE];

  const TileJob job = locate_tile<BM, BN>(p);
  const bf16* __restrict__ A = job.a;
  const bf16* __restrict__ B = job.b;
  const int M = job.m, N = p.n, tm = job.tm, tn = job.tn;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS targets stay scalar
  const int wm = w / WGN, wn = w % WGN;

  // per-lane global offsets of the chunks this lane fetches (32-bit; host checks the range)
  const int ld_r = lane / CPR;
  const int ld_p = lane % CPR;
  int a_off[A_LOADS], b_off[B_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int r = (w * A_LOADS + i) * RPL + ld_r;
    a_off[i] = min(tm * BM + r, M - 1) * static_cast<int>(p.lda) + 8 * (ld_p ^ swz<BK>(r));
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int r = (w * B_LOADS + i) * RPL + ld_r;
    b_off[i] = min(tn * BN + r, N - 1) * static_cast<int>(p.ldb) + 8 * (ld_p ^ swz<BK>(r));
  }
  // The LPW loads of one K tile form PARTS parts (load j belongs to part j % PARTS, A loads
  // numbered before B loads) so that they can be spread over several k-steps.
  // buffer loads straight to LDS: a 32-bit VGPR byte offset per load, the K position in an SGPR
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, M * static_cast<int>(p.lda) * 2, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rsrc_b =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, N * static_cast<int>(p.ldb) * 2, kBufferFlags);
  auto issue = [&](int kt, int stage, int part) {  // part < 0: all loads
    bf16* sa = lds + stage * STAGE;
    bf16* sb = sa + A_STAGE;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      if (part < 0 || i % PARTS == part)
        buffer_load_lds16(rsrc_a, sa + (w * A_LOADS + i) * RPL * BK, a_off[i] * 2, kt * BK * 2);
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      if (part < 0 || (A_LOADS + i) % PARTS == part)
        buffer_load_lds16(rsrc_b, sb + (w * B_LOADS + i) * RPL * BK, b_off[i] * 2, kt * BK * 2);
  };


  // fragment reads: row r, logical chunk 2 ks + g, stored at chunk (2 ks + g) ^ swz(r)
  int a_row[FM], b_row[FN];
#pragma unroll
  for (int j = 0; j < FM; ++j) a_row[j] = wm * WM + j * 32 + l32;
#pragma unroll
  for (int i = 0; i < FN; ++i) b_row[i] = wn * WN + i * 32 + l32;
  bf16x8 wf[2][FN], xf[2][FM];
  auto read_frags = [&](int stage, int ks, int buf) {
    const bf16* sa = lds + stage * STAGE;
    const bf16* sb = sa + A_STAGE;
    const int c = 2 * ks + g;
#pragma unroll
    for (int i = 0; i < FN; ++i)
      wf[buf][i] = *reinterpret_cast<const bf16x8*>(sb + b_row[i] * BK + 8 * (c ^ swz<BK>(b_row[i])));
#pragma unroll
    for (int j = 0; j < FM; ++j)
      xf[buf][j] = *reinterpret_cast<const bf16x8*>(sa + a_row[j] * BK + 8 * (c ^ swz<BK>(a_row[j])));
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};

  // Software pipeline: the fragments of the next k-step are read from LDS while the MFMAs
  // of the current one run; the wait + barrier for K tile kt+1 sits before the last k-step
  // of tile kt, whose fragments are already in registers, so the stage being retired can be
  // refilled right after that barrier. The refill of tile kt+STAGES starts there (part 0)
  // and continues over the first PARTS-1 k-steps of tile kt+1 (parts 1..), so that the
  // eight waves do not queue all their loads at the same moment.
  const int KT = p.k / BK;
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s, s, -1);
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  issue(min(STAGES - 1, KT - 1), STAGES - 1, 0);
  read_frags(0, 0, 0);

  auto mfmas = [&](int cur) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[cur][i], xf[cur][j], acc[i][j], 0, 0, 0);
  };
  constexpr int NR = FN + FM, NM = FN * FM;
  constexpr int L0 = part_loads(LPW, PARTS, 0), L1 = part_loads(LPW, PARTS, 1);
  constexpr int L2 = part_loads(LPW, PARTS, 2), L3 = part_loads(LPW, PARTS, 3);

  // Every K tile but the last: branch-free, so each k-step is one scheduling region. Refills
  // always issue; past the end they reload the final K tile into a retired stage that no
  // pending tile occupies and nothing reads again (the loads are drained before the
  // epilogue reuses the ring). Loads issued after tile kt+1's last part number
  // (STAGES - 2) * LPW at the wait of tile kt, for every PARTS.
  for (int kt = 0; kt + 1 < KT; ++kt) {
    const int stage = kt % STAGES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) {
        read_frags(stage, ks + 1, cur ^ 1);
        if (ks + 1 < PARTS) issue(min(kt + STAGES - 1, KT - 1), (kt + STAGES - 1) % STAGES, ks + 1);
        mfmas(cur);
        if (ks + 1 >= PARTS)
          order_kstep<NR, NM, 0>();
        else if (ks == 0)
          order_kstep<NR, NM, L1>();
        else if (ks == 1)
          order_kstep<NR, NM, L2>();
        else
          order_kstep<NR, NM, L3>();
      } else {
        // tile kt+1 has landed (loads issued after it may still fly) and this wave's
        // fragment reads of stage kt are done before the barrier lets the stage be refilled;
        // the wait stays behind the previous k-step's MFMAs, which cover it
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_lgkm0<(STAGES - 2) * LPW>();
        __builtin_amdgcn_s_barrier();
        read_frags((kt + 1) % STAGES, 0, cur ^ 1);
        issue(min(kt + STAGES, KT - 1), stage, 0);
        mfmas(cur);
        order_kstep<NR, NM, L0>();
      }
    }
  }
  {  // last K tile
    const int stage = (KT - 1) % STAGES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) read_frags(stage, ks + 1, cur ^ 1);
      mfmas(cur);
      if (ks + 1 < KS) order_kstep<NR, NM, 0>();
    }
  }
  wait_vmcnt<0>();

  store_tile<BM, BN, WM, WN, FM, FN, NW, STAGES * STAGE, EPI, TC>(acc, lds, job, N, p.ldc, wm, wn, p.qk, [] {});
}

// Instruction order of one k-step of gemm_w4_kernel: an MFMA, then the next k-step's NR
// fragment reads each followed by an MFMA, then W LDS writes and L global loads dealt over the
// remaining MFMAs as evenly as they go (the first slots take one more of each when they do not
// divide), then the MFMAs left over.
template <int W, int L, int R, int... S>
__device__ __forceinline__ void order_w4_slots(std::integer_sequence<int, S...>) {
  (([] {
     constexpr int w = W / R + (S < W % R ? 1 : 0);
     constexpr int l = L / R + (S < L % R ? 1 : 0);
     if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);  // DS write
     if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);  // VMEM read
     __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
   }()),
   ...);
}

template <int NR, int NM, int W, int L>
__device__ __forceinline__ void order_w4() {
  constexpr int R = NM - 1 - NR;  // MFMAs after the fragment reads
  static_assert(R > 0 && W <= 2 * R && L <= 2 * R, "MFMAs per k-step");
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
  order_w4_slots<W, L, R>(std::make_integer_sequence<int, R>{});
}

// Four waves (one per SIMD) in a 2 x 2 grid over a BM x 256 tile, each owning a (BM/2) x 128
// block (128 x 128 for BM = 256, 96 x 128 for BM = 192), with register-staged refills: every
// wave loads its quarter of K tile t + 2 from global memory into registers (16-byte loads that
// do not hold up the wave, unlike global_load_lds) while it multiplies tile t, and writes tile
// t + 1, loaded one K tile earlier, into the free LDS stage. A 128-wide block per wave reads
// fewer LDS bytes per MFMA than the eight-wave kernel's 128 x 64; the accumulators live in the
// AGPRs. Inside each k-step the fragment reads of the next k-step, then this k-step's share of
// the LDS writes and global loads, are spread between the MFMAs.
template <int BM, int EPI, typename TC, bool PERSIST>
__global__ __launch_bounds__(256) void gemm_w4_kernel(GemmArgs p) {
  constexpr int BN = 256, BK = 64, NW = 4;
  constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
  constexpr int KS = BK / 16;
  constexpr int CPR = BK / 8;
  constexpr int RPL = 64 / CPR;                // rows per 1 KB wave load
  constexpr int A_LOADS = BM / RPL / NW;       // 8 (BM = 256) or 6 (BM = 192)
  constexpr int B_LOADS = BN / RPL / NW;       // 8
  constexpr int LW = A_LOADS + B_LOADS;        // loads of 16 bytes per lane per K tile
  constexpr int NR = FN + FM, NM = FN * FM;    // fragment reads and MFMAs per k-step
  constexpr int A_STAGE = BM * BK, STAGE = (BM + BN) * BK;
  static_assert(KS == 4 && BM % 64 == 0 && A_LOADS * RPL * NW == BM, "tile / wave split");
  // the LW loads of a K tile are dealt over the 4 k-steps at G0..G3 (boundaries), its LDS
  // writes over the first three at W0, W1
  constexpr int G1 = (LW + 3) / 4, G2 = (2 * LW + 3) / 4, G3 = (3 * LW + 3) / 4;
  constexpr int W0 = (LW + 2) / 3, W1 = (2 * LW + 2) / 3;
  static_assert(W0 >= G1 && W1 >= G2, "a slot is written to LDS before it is reloaded");
  __shared__ __attribute__((aligned(1024))) bf16 lds[2 * STAGE];

  int cur_tile = persistent_tile(p, 0);
  if (cur_tile < 0) return;
  TileJob job = locate_tile_at<BM, BN>(p, cur_tile);
  const int N = p.n;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;

  // load i: A rows (8 w + i) * RPL .. + RPL for i < 8, B rows (8 w + i - 8) * RPL .. for the rest;
  // lane l fetches the chunk that belongs at byte 16 l of that 1 KB block in LDS
  const int ld_r = lane / CPR;
  const int ld_p = lane % CPR;
  int off[LW];
  auto set_offsets = [&](const TileJob& jb) {
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const bool is_a = i < A_LOADS;
      const int r = (is_a ? w * A_LOADS + i : w * B_LOADS + i - A_LOADS) * RPL + ld_r;
      off[i] = is_a ? min(jb.tm * BM + r, jb.m - 1) * static_cast<int>(p.lda) + 8 * (ld_p ^ swz<BK>(r))
                    : min(jb.tn * BN + r, N - 1) * static_cast<int>(p.ldb) + 8 * (ld_p ^ swz<BK>(r));
    }
  };
  set_offsets(job);
  auto dst = [&](int i) {  // element offset inside a stage
    return (i < A_LOADS ? (w * A_LOADS + i) * RPL * BK : A_STAGE + (w * B_LOADS + i - A_LOADS) * RPL * BK) + 8 * lane;
  };
  // one register slot per load: slot i of K tile t + 1 is written to LDS before slot i of
  // K tile t + 2 is loaded into it
  bf16x8 staged[LW];
  // buffer loads: the per-load 32-bit byte offset is the only VGPR an address costs, the K
  // position goes in an SGPR, and reads past the operand return zeros instead of faulting
  __amdgpu_buffer_rsrc_t rsrc_a, rsrc_b;
  auto set_rsrc = [&](const TileJob& jb) {
    rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void*)jb.a, (short)0, jb.m * static_cast<int>(p.lda) * 2, kBufferFlags);
    rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void*)jb.b, (short)0, N * static_cast<int>(p.ldb) * 2, kBufferFlags);
  };
  set_rsrc(job);
  auto gload = [&](int kt, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
      staged[i] = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(i < A_LOADS ? rsrc_a : rsrc_b, off[i] * 2, kt * BK * 2, 0));
  };
  auto lwrite = [&](int stage, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) *reinterpret_cast<bf16x8*>(lds + stage * STAGE + dst(i)) = staged[i];
  };

  int a_row[FM], b_row[FN];
#pragma unroll
  for (int j = 0; j < FM; ++j) a_row[j] = wm * WM + j * 32 + l32;
#pragma unroll
  for (int i = 0; i < FN; ++i) b_row[i] = wn * WN + i * 32 + l32;
  bf16x8 wf[2][FN], xf[2][FM];
  auto read_frags = [&](int stage, int ks, int buf) {
    const bf16* sa = lds + stage * STAGE;
    const bf16* sb = sa + A_STAGE;
    const int c = 2 * ks + g;
#pragma unroll
    for (int i = 0; i < FN; ++i)
      wf[buf][i] = *reinterpret_cast<const bf16x8*>(sb + b_row[i] * BK + 8 * (c ^ swz<BK>(b_row[i])));
#pragma unroll
    for (int j = 0; j < FM; ++j)
      xf[buf][j] = *reinterpret_cast<const bf16x8*>(sa + a_row[j] * BK + 8 * (c ^ swz<BK>(a_row[j])));
  };
  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};
  auto mfmas = [&](int cur) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[cur][i], xf[cur][j], acc[i][j], 0, 0, 0);
  };

  // K tile t: multiplied from LDS stage t % 2. Its first three k-steps write tile t + 1
  // (loaded during tile t - 1) into stage (t + 1) % 2, six, five and five 1 KB blocks; its
  // four k-steps load a quarter of tile t + 2 each into slots already written. The barrier
  // before the last k-step publishes the writes and retires stage t % 2. Past the end the
  // loads repeat the last K tile; nothing writes them to LDS.
  const int KT = p.k / BK;
  gload(0, 0, LW);
  for (int round = 0;; ++round) {
  lwrite(0, 0, LW);  // K tile 0, loaded before the previous tile's epilogue (or just above)
  gload(min(1, KT - 1), 0, LW);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __syncthreads();
  read_frags(0, 0, 0);

  auto ktile = [&](int t, auto P) {  // t + 1 < KT, P = t % 2 as a compile-time constant
    constexpr int S = decltype(P)::value;
    const int t2 = min(t + 2, KT - 1);
    // k-step 0
    read_frags(S, 1, 1);
    lwrite(S ^ 1, 0, W0);
    gload(t2, 0, G1);
    mfmas(0);
    order_w4<NR, NM, W0, G1>();
    // k-step 1
    read_frags(S, 2, 0);
    lwrite(S ^ 1, W0, W1);
    gload(t2, G1, G2);
    mfmas(1);
    order_w4<NR, NM, W1 - W0, G2 - G1>();
    // k-step 2
    read_frags(S, 3, 1);
    lwrite(S ^ 1, W1, LW);
    gload(t2, G2, G3);
    mfmas(0);
    order_w4<NR, NM, LW - W1, G3 - G2>();
    // k-step 3: publish tile t + 1, then read its first fragments behind the last MFMAs
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes and reads are done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(S ^ 1, 0, 0);
    gload(t2, G3, LW);
    mfmas(1);
    order_w4<NR, NM, 0, LW - G3>();
  };
  int t = 0;
  for (; t + 2 < KT; t += 2) {
    ktile(t, std::integral_constant<int, 0>{});
    ktile(t + 1, std::integral_constant<int, 1>{});
  }
  if (t + 1 < KT) {
    ktile(t, std::integral_constant<int, 0>{});
    ++t;
  }
  {  // last K tile, stage t % 2
    const int S = t & 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) read_frags(S, ks + 1, cur ^ 1);
      mfmas(cur);
    }
  }
  wait_vmcnt<0>();  // the repeated loads of the last K tile
  // the next tile's first K tile is in flight while this tile's output goes out
  const int next_tile = PERSIST ? persistent_tile(p, round + 1) : -1;
  const TileJob next = next_tile >= 0 ? locate_tile_at<BM, BN>(p, next_tile) : job;
  store_tile<BM, BN, WM, WN, FM, FN, NW, 2 * STAGE, EPI, TC>(acc, lds, job, N, p.ldc, wm, wn, p.qk, [&] {
    if (next_tile >= 0) {
      set_rsrc(next);
      set_offsets(next);
      gload(0, 0, LW);
    }
  });
  if (next_tile < 0) break;
  __syncthreads();  // every wave is done with the staged output before stage 0 is rewritten
  job = next;
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x16{};
  }
}

// Epilogue of the 16 x 16 x 32 MFMA layout: acc[i][j][e] = C[m, n] with n = tile + wave col +
// 16 i + 4 (lane / 16) + e, m = tile + wave row + 16 j + lane % 16. SwiGLU: in every 64-row
// group of the packed weight the first 32 rows are w1 and the next 32 w3, so acc[i] (i % 4 < 2)
// pairs with acc[i + 2] in the same lane, output column 32 (group) + 16 (i % 4) + 4 (lane / 16)
// + e. BF16 output is staged through the LDS ring and leaves in 16-byte row chunks: rows of 160
// outputs (80 dwords, so rows r and r + 4 would share banks) padded by 16 bytes, rows of 128 or
// 256 (whose padded tile would not fit the ring) with 4-element unit u of row r at
// u ^ 2 (r & 15), as store_tile. FP32 output is stored straight from the registers. `mid` as in
// store_tile.
template <int BM, int BN, int WM, int WN, int FM, int FN, int NW, int RING, int EPI, typename TC, typename Mid>
__device__ __forceinline__ void store_tile16(f32x4 (&acc)[FN][FM], bf16* lds, const TileJob& job, int N, long ldc,
                                             int wm, int wn, const QkRope& qk, Mid&& mid) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int M = job.m, tm = job.tm, tn = job.tn;
  const float* __restrict__ bias = job.bias;
  TC* __restrict__ C = static_cast<TC*>(job.c);
  constexpr bool SWIGLU = EPI == IRIS_EPI_SILU_MUL;
  static_assert(!SWIGLU || WN % 64 == 0, "SwiGLU pairs 32-column blocks inside one wave");
  constexpr int OUT_N = SWIGLU ? BN / 2 : BN;  // output columns of the tile
  const int n_out = SWIGLU ? N / 2 : N;
  // tile-local output column of acc[i][.][0]
  auto col = [&](int i) {
    return SWIGLU ? 32 * ((wn * WN) / 64 + i / 4) + 16 * (i % 4) + 4 * q4 : wn * WN + 16 * i + 4 * q4;
  };
  // the four outputs of acc[i][j] (bias: the FP32 bias of those columns, zeros without one)
  auto value = [&](int i, int j, int e, float bv) {
    if constexpr (SWIGLU)
      return silu(acc[i][j][e]) * acc[i + 2][j][e];
    else
      return acc[i][j][e] + bv;
  };
  if constexpr (sizeof(TC) == 2) {
    constexpr bool SWZ = (OUT_N / 4) % 32 == 0;
    constexpr int PITCH = SWZ ? OUT_N : OUT_N + 8;
    static_assert(BM * PITCH <= RING, "output tile must fit in the LDS ring");
    bf16* cl = lds;
    __syncthreads();
    __shared__ float qk_gain[EPI == kEpiQkRope ? 256 : 1];
    [[maybe_unused]] f32x4 qk_cos[EPI == kEpiQkRope ? 16 : 1], qk_sin[EPI == kEpiQkRope ? 16 : 1];
    if constexpr (EPI == kEpiQkRope) {
      static_assert(BM == 64 * NW && BN == 256 && SWZ, "one 256-wide tile row per thread");
      qk_tables<BM>(job, qk, qk_gain, qk_cos, qk_sin);
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int r = wm * WM + 16 * j + l16;
      bf16* crow_l = cl + r * PITCH;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        if (SWIGLU && i % 4 >= 2) continue;
        const int nl = col(i);
        f32x4 bv = {};
        if (!SWIGLU && bias) bv = load4(bias + min(tn * BN + nl, N - 4));
        store_out4(crow_l + (SWZ ? 4 * ((nl / 4) ^ (2 * (r & 15))) : nl), value(i, j, 0, bv[0]), value(i, j, 1, bv[1]),
                   value(i, j, 2, bv[2]), value(i, j, 3, bv[3]));
      }
    }
    __syncthreads();
    mid();
    if constexpr (EPI == kEpiQkRope) {
      qk_store<BM, NW>(cl, job, N, ldc, qk, qk_gain, qk_cos, qk_sin);
      return;
    }
    constexpr int CHUNKS = OUT_N / 8;
    const int col0 = tn * OUT_N;
#pragma unroll 4
    for (int idx = tid; idx < BM * CHUNKS; idx += 64 * NW) {
      const int r = idx / CHUNKS;
      const int c = idx - r * CHUNKS;
      const int m = tm * BM + r;
      const int n0 = col0 + 8 * c;
      if (m >= M || n0 >= n_out) continue;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(cl + r * PITCH + 8 * (SWZ ? c ^ (r & 15) : c));
      TC* dst = C + static_cast<long>(m) * ldc + n0;
      if (n0 + 8 <= n_out) {
        // streamed (nontemporal): the whole output goes out in the tile's last microseconds; with
        // it the launches end sooner (2% per SwiGLU call, 1.4% over all GEMM launches, eager)
        __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(dst));
      } else {
        *reinterpret_cast<bf16x4*>(dst) = bf16x4{v[0], v[1], v[2], v[3]};  // n_out % 4 == 0
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = tm * BM + wm * WM + 16 * j + l16;
    if (m >= M) continue;
    TC* crow = C + static_cast<long>(m) * ldc + tn * OUT_N;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      if (SWIGLU && i % 4 >= 2) continue;
      const int nl = col(i);
      if (tn * OUT_N + nl >= n_out) continue;
      f32x4 bv = {};
      if (!SWIGLU && bias) bv = load4(bias + tn * BN + nl);
      store_out4(crow + nl, value(i, j, 0, bv[0]), value(i, j, 1, bv[1]), value(i, j, 2, bv[2]), value(i, j, 3, bv[3]));
    }
  }
  mid();
}

// v_mfma_f32_16x16x32_bf16 accumulating in place, c += a b. Written as inline assembly: with the
// builtin, the register allocator rotates the 40 to 64 four-register accumulator tuples of
// gemm_w4h_kernel between registers inside the K loop (hundreds of accumulator moves per K
// tile). An asm statement is also an ordering point for memory operations, so the LDS reads and
// writes and the global loads between these MFMAs issue where the source places them. The
// compiler pads no hazards for instructions it does not know to be MFMAs; the only ones it can
// create are at the edges of straight-line MFMA runs, where it may zero or copy accumulators:
// BEFORE pads a VALU write of an accumulator ahead of the run's first MFMA (5 wait states, more
// than the 2 needed), AFTER pads a VALU read or write of the last MFMA's result behind it (24
// wait states: 4 passes of 4 cycles plus the write-back). Inside a run every MFMA accumulates
// into a tuple no other instruction touches, and a tuple's next MFMA is dozens of MFMAs later.
template <bool BEFORE, bool AFTER>
__device__ __forceinline__ void mfma16_acc(f32x4& c, const bf16x8& a, const bf16x8& b) {
  // (the scheduling barriers keep the compiler from moving a VALU access of an accumulator
  // into the run: asm statements order memory operations only)
  if constexpr (BEFORE) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 4\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  } else if constexpr (AFTER) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n\ts_nop 15\n\ts_nop 7" : "+a"(c) : "v"(a), "v"(b));
    __builtin_amdgcn_sched_barrier(0);
  } else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// Four waves (one per SIMD) in a 2 x 2 grid over a BM x BN tile on v_mfma_f32_16x16x32_bf16,
// refilled as gemm_w4_kernel refills (K tile t + 2 loaded into registers while tile t is
// multiplied, tile t + 1 written from them into the free LDS stage); plain, bias, SwiGLU and
// q|k|v-store epilogues. Besides 256 x 256 and 192 x 256, the 16-row granularity of this MFMA
// admits tiles the 32 x 32 one does not: 288 x 160 and 256 x 160 cut a 2560-column output at
// 4352 and 4096 rows into 256 tiles (16 x 16; 192 x 256 tiles leave 26 of 256 CUs idle there),
// 128 x 160 cuts 4096 x 1280 into 256. A K tile of 64 is two k-steps of 32. In
// k-step 0 each of the first NR MFMAs is followed by one fragment read of k-step 1, the next
// ones alternately by an LDS write of the first half of tile t + 1 and the load of tile t + 2
// into the slot just written. In k-step 1 the second half follows the same way, then the wait
// and barrier that publish tile t + 1 and retire stage t % 2, then one read of tile t + 1's
// first fragments after each MFMA.
// Bytes of gemm_w4h_tiles' LDS ring: two stages of BM x 64 and BN x 64 operand tiles (the output
// staging of the store reuses it). The ring is the launch's dynamic LDS, so that a kernel running
// two tile shapes holds one ring; the compiler also keeps the constant parts of the fragment and
// refill addresses as instruction offsets there (a static array reached through a pointer or a
// helper function cost one address register per access, and spills in the 256 x 256 kernels).
template <int BM, int BN>
constexpr unsigned w4h_lds_bytes() {
  return 2u * (BM + BN) * 64u * sizeof(bf16);
}

// The body of gemm_w4h_kernel for workgroup wg of nwg (wg on XCD wg % 8).
template <int BM, int BN, int EPI, typename TC, bool PERSIST>
__device__ __forceinline__ void gemm_w4h_tiles(const GemmArgs& p, const int wg, const int nwg) {
  constexpr int BK = 64, NW = 4;
  constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
  constexpr int CPR = BK / 8;
  constexpr int RPL = 64 / CPR;                // rows per 1 KB wave load
  constexpr int A_LOADS = BM / RPL / NW;
  constexpr int B_LOADS = BN / RPL / NW;
  constexpr int LW = A_LOADS + B_LOADS;        // loads of 16 bytes per lane per K tile
  constexpr int NR = FN + FM, NM = FN * FM;    // fragment reads and MFMAs per k-step
  constexpr int A_STAGE = BM * BK, STAGE = (BM + BN) * BK;
  static_assert(WM % 16 == 0 && WN % 16 == 0 && A_LOADS * RPL * NW == BM && B_LOADS * RPL * NW == BN,
                "tile / wave split");
  static_assert(EPI == IRIS_EPI_NONE || EPI == IRIS_EPI_SILU_MUL || EPI == kEpiQkRope,
                "plain, bias, SwiGLU or q|k|v epilogue");
  constexpr int W0 = (LW + 1) / 2;             // slots written to LDS (and reloaded) in k-step 0
  constexpr int W1 = LW - W0;                  // the rest, in k-step 1 before its barrier
  static_assert(NR + 2 * W0 <= NM && 2 * W1 + NR < NM && W1 > 0, "MFMAs per k-step");
  static_assert(2 * STAGE * sizeof(bf16) == w4h_lds_bytes<BM, BN>(), "LDS ring");
  extern __shared__ __attribute__((aligned(1024))) bf16 lds[];  // w4h_lds_bytes<BM, BN>() at launch

  int cur_tile = persistent_tile(p, 0, wg, nwg);
  if (cur_tile < 0) return;
  TileJob job = locate_tile_at<BM, BN>(p, cur_tile);
  const int N = p.n;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  // load i: A rows (w A_LOADS + i) RPL .. + RPL for i < A_LOADS, B rows (w B_LOADS + i -
  // A_LOADS) RPL .. for the rest; lane l fetches the chunk that belongs at byte 16 l of that
  // 1 KB block in LDS. Byte offset of load j of an operand: a per-lane part shared by the loads
  // of the same parity (a row's swizzle depends on (row / 2) % 8, and j + 2 is 16 rows further),
  // plus (j & ~1) RPL rows and the K position in an SGPR: four address VGPRs instead of one per
  // load. Rows past an operand's end are not clamped: the buffer's range check returns zeros
  // (or, past 2^32 bytes, wraps inside the buffer), which reach only output rows and columns
  // that are not stored.
  const int ld_r = lane / CPR;
  const int ld_p = lane % CPR;
  const unsigned lda2 = 2u * static_cast<unsigned>(p.lda), ldb2 = 2u * static_cast<unsigned>(p.ldb);
  unsigned voff[2][2];  // [operand][parity]
  auto set_offsets = [&](const TileJob& jb) {
#pragma unroll
    for (int op = 0; op < 2; ++op)
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int r = (w * (op ? B_LOADS : A_LOADS) + par) * RPL + ld_r;  // row inside the tile
        const unsigned row = static_cast<unsigned>((op ? jb.tn * BN : jb.tm * BM) + r);
        voff[op][par] = row * (op ? ldb2 : lda2) + 16u * static_cast<unsigned>(ld_p ^ swz<BK>(r));
      }
  };
  set_offsets(job);
  bf16x8 staged[LW];
  __amdgpu_buffer_rsrc_t rsrc_a, rsrc_b;
  auto set_rsrc = [&](const TileJob& jb) {
    rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void*)jb.a, (short)0, jb.m * static_cast<int>(p.lda) * 2, kBufferFlags);
    rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void*)jb.b, (short)0, N * static_cast<int>(p.ldb) * 2, kBufferFlags);
  };
  set_rsrc(job);
  auto load1 = [&](int kt, int i) {
    const int op = i < A_LOADS ? 0 : 1;
    const int j = op ? i - A_LOADS : i;
    const unsigned soff =
        static_cast<unsigned>(kt * BK * 2) + static_cast<unsigned>((j & ~1) * RPL) * (op ? ldb2 : lda2);
    staged[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(op ? rsrc_b : rsrc_a, voff[op][j & 1],
                                                                                static_cast<int>(soff), 0));
  };
  auto write1 = [&](int stage, int i) {
    bf16* blk = lds + stage * STAGE +
                (i < A_LOADS ? (w * A_LOADS + i) * RPL * BK : A_STAGE + (w * B_LOADS + i - A_LOADS) * RPL * BK);
    *reinterpret_cast<bf16x8*>(blk + 8 * lane) = staged[i];
  };

  // a 16-row fragment: lane l reads row l % 16 of the block, logical chunk 4 ks + l / 16 (the
  // blocks start at multiples of 16 rows, so the swizzle depends on the lane only)
  int frag_off[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) frag_off[ks] = l16 * BK + 8 * ((4 * ks + q4) ^ swz<BK>(l16));
  bf16x8 wf[2][FN], xf[2][FM];
  // read r of a k-step: weight fragment r (r < FN), else activation fragment r - FN
  auto read1 = [&](int stage, int ks, int buf, int r) {
    const bf16* s = lds + stage * STAGE + frag_off[ks];
    if (r < FN)
      wf[buf][r] = *reinterpret_cast<const bf16x8*>(s + A_STAGE + (wn * WN + 16 * r) * BK);
    else
      xf[buf][r - FN] = *reinterpret_cast<const bf16x8*>(s + (wm * WM + 16 * (r - FN)) * BK);
  };
  f32x4 acc[FN][FM];
  auto zero_acc = [&] {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{};
  };
  zero_acc();
  using T = std::true_type;
  using F = std::false_type;
  // MFMA idx of a k-step (row-major over the FN x FM tuples) from fragment buffer buf
  auto mfma = [&](int buf, int idx, auto before, auto after) {
    mfma16_acc<decltype(before)::value, decltype(after)::value>(acc[idx / FM][idx % FM], wf[buf][idx / FM],
                                                                 xf[buf][idx % FM]);
  };

  // K tile t (t + 1 < KT) from stage S; FIRST / LAST: it opens / closes a straight-line run
  auto ktile = [&](int t, auto S_, auto first_, auto last_) {
    constexpr int S = decltype(S_)::value;
    const int t2 = min(t + 2, p.k / BK - 1);
#pragma unroll
    for (int idx = 0; idx < NM; ++idx) {
      if (idx == 0 && decltype(first_)::value)
        mfma(0, idx, T{}, F{});
      else
        mfma(0, idx, F{}, F{});
      if (idx < NR) {
        read1(S, 1, 1, idx);
      } else if (idx < NR + 2 * W0) {
        const int q = (idx - NR) / 2;
        if ((idx - NR) % 2 == 0)
          write1(S ^ 1, q);
        else
          load1(t2, q);
      }
    }
#pragma unroll
    for (int idx = 0; idx < NM; ++idx) {
      if (idx == NM - 1 && decltype(last_)::value)
        mfma(1, idx, F{}, T{});
      else
        mfma(1, idx, F{}, F{});
      if (idx < 2 * W1) {
        const int q = W0 + idx / 2;
        if (idx % 2 == 0) {
          write1(S ^ 1, q);
        } else {
          load1(t2, q);
          if (idx == 2 * W1 - 1) {
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes and reads are done
            __builtin_amdgcn_s_barrier();
          }
        }
      } else if (idx < 2 * W1 + NR) {
        read1(S ^ 1, 0, 0, idx - 2 * W1);
      }
    }
  };

  const int KT = p.k / BK;
#pragma unroll
  for (int i = 0; i < LW; ++i) load1(0, i);
  for (int round = 0;; ++round) {
#pragma unroll
  for (int i = 0; i < LW; ++i) write1(0, i);  // K tile 0, loaded before the previous tile's epilogue (or above)
#pragma unroll
  for (int i = 0; i < LW; ++i) load1(min(1, KT - 1), i);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __syncthreads();
#pragma unroll
  for (int r = 0; r < NR; ++r) read1(0, 0, 0, r);

  int t = 0;
  for (; t + 2 < KT; t += 2) {
    ktile(t, std::integral_constant<int, 0>{}, T{}, F{});
    ktile(t + 1, std::integral_constant<int, 1>{}, F{}, T{});
  }
  if (t + 1 < KT) {
    ktile(t, std::integral_constant<int, 0>{}, T{}, T{});
    ++t;
  }
  {  // last K tile, stage t % 2 (its k-step 1 fragments read between k-step 0's MFMAs)
    const int S = t & 1;
#pragma unroll
    for (int idx = 0; idx < NM; ++idx) {
      if (idx == 0)
        mfma(0, idx, T{}, F{});
      else
        mfma(0, idx, F{}, F{});
      if (idx < NR) read1(S, 1, 1, idx);
    }
#pragma unroll
    for (int idx = 0; idx < NM; ++idx) {
      if (idx == NM - 1)
        mfma(1, idx, F{}, T{});
      else
        mfma(1, idx, F{}, F{});
    }
  }
  wait_vmcnt<0>();  // the repeated loads of the last K tile
  const int next_tile = PERSIST ? persistent_tile(p, round + 1, wg, nwg) : -1;
  const TileJob next = next_tile >= 0 ? locate_tile_at<BM, BN>(p, next_tile) : job;
  store_tile16<BM, BN, WM, WN, FM, FN, NW, 2 * STAGE, EPI, TC>(acc, lds, job, N, p.ldc, wm, wn, p.qk, [&] {
    if (next_tile >= 0) {
      set_rsrc(next);
      set_offsets(next);
#pragma unroll
      for (int i = 0; i < LW; ++i) load1(0, i);
    }
  });
  if (next_tile < 0) break;
  __syncthreads();  // every wave is done with the staged output before stage 0 is rewritten
  job = next;
  zero_acc();
  }
}

template <int BM, int BN, int EPI, typename TC, bool PERSIST>
__global__ __launch_bounds__(256) void gemm_w4h_kernel(GemmArgs p) {
  gemm_w4h_tiles<BM, BN, EPI, TC, PERSIST>(p, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
}

// Two independent GEMMs in one grid, one tile per workgroup, BF16 outputs: workgroups
// [0, p1.total_tiles) run the first, the second starts at the next multiple of 8 (the workgroups
// between exit at once), so each keeps the XCD mapping of a launch of its own. Against two
// launches it saves the boundary between them (the first one's last output writes and the
// second one's first K tiles overlap on the CUs that finish first).
template <int BM1, int BN1, int EPI1, int BM2, int BN2, int EPI2>
__global__ __launch_bounds__(256) void gemm_w4h_pair_kernel(GemmArgs p1, GemmArgs p2) {
  const int wg = static_cast<int>(blockIdx.x);
  const int second = (p1.total_tiles + 7) & ~7;
  if (wg < second) {
    if (wg < p1.total_tiles) gemm_w4h_tiles<BM1, BN1, EPI1, bf16, false>(p1, wg, p1.total_tiles);
  } else {
    gemm_w4h_tiles<BM2, BN2, EPI2, bf16, false>(p2, wg - second, p2.total_tiles);
  }
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int PARTS>
int launch_tile(GemmArgs& args, int c_dtype, int epilogue, hipStream_t stream) {
  const dim3 grid(args.total_tiles);
  const dim3 block(64 * WGM * WGN);
  if (epilogue == IRIS_EPI_SILU_MUL) {
    // the SwiGLU epilogue pairs 32-column blocks inside one wave: an even count per wave
    if constexpr ((BN / WGN / 32) % 2 == 0) {
      if (c_dtype == IRIS_BF16)
        gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_SILU_MUL, bf16><<<grid, block, 0, stream>>>(args);
      else
        gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_SILU_MUL, float><<<grid, block, 0, stream>>>(args);
    } else {
      return fail(IRIS_E_UNSUPPORTED, "gemm: tile %dx%d has no SwiGLU epilogue", BM, BN);
    }
  } else if (epilogue == IRIS_EPI_SILU) {
    if (c_dtype == IRIS_BF16)
      gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_SILU, bf16><<<grid, block, 0, stream>>>(args);
    else
      gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_SILU, float><<<grid, block, 0, stream>>>(args);
  } else {
    if (c_dtype == IRIS_BF16)
      gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_NONE, bf16><<<grid, block, 0, stream>>>(args);
    else
      gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, PARTS, IRIS_EPI_NONE, float><<<grid, block, 0, stream>>>(args);
  }
  return check_launch("gemm_bf16");
}


// Plain BF16 output runs persistently (one workgroup per CU, the next tile's first K tile
// loaded while the current tile is stored); the SwiGLU and FP32 epilogues keep one tile per
// workgroup, since the register allocator spills inside the K loop when their epilogue shares
// the persistent loop with it.
template <int BM>
int launch_w4(GemmArgs& args, int c_dtype, int epilogue, hipStream_t stream) {
  if (epilogue == IRIS_EPI_SILU) return fail(IRIS_E_UNSUPPORTED, "gemm: the four-wave tile has no SiLU epilogue");
  const int cus = device_cus();
  const dim3 all(args.total_tiles);
  if (epilogue == IRIS_EPI_SILU_MUL) {
    if (c_dtype == IRIS_BF16)
      gemm_w4_kernel<BM, IRIS_EPI_SILU_MUL, bf16, false><<<all, 256, 0, stream>>>(args);
    else
      gemm_w4_kernel<BM, IRIS_EPI_SILU_MUL, float, false><<<all, 256, 0, stream>>>(args);
  } else if (epilogue == kEpiQkRope) {
    // one tile per workgroup: the next tile's loads in flight would spill the store's registers
    if constexpr (BM == 256)
      gemm_w4_kernel<BM, kEpiQkRope, bf16, false><<<all, 256, 0, stream>>>(args);
    else
      return fail(IRIS_E_UNSUPPORTED, "gemm: the q|k|v store runs on 256 x 256 tiles");
  } else {
    if (c_dtype == IRIS_BF16)
      gemm_w4_kernel<BM, IRIS_EPI_NONE, bf16, true><<<dim3(args.total_tiles < cus ? args.total_tiles : cus), 256, 0,
                                                       stream>>>(args);
    else
      gemm_w4_kernel<BM, IRIS_EPI_NONE, float, false><<<all, 256, 0, stream>>>(args);
  }
  return check_launch("gemm_bf16");
}

template <int BM, int BN>
int launch_w4h(GemmArgs& args, int c_dtype, int epilogue, hipStream_t stream) {
  if (epilogue == IRIS_EPI_SILU) return fail(IRIS_E_UNSUPPORTED, "gemm: the four-wave tiles have no SiLU epilogue");
  const dim3 all(args.total_tiles);
  if (epilogue == IRIS_EPI_SILU_MUL) {
    // one tile per workgroup, as gemm_w4_kernel's SwiGLU form
    if constexpr (BN / 2 % 64 == 0) {
      if (c_dtype == IRIS_BF16)
        gemm_w4h_kernel<BM, BN, IRIS_EPI_SILU_MUL, bf16, false><<<all, 256, w4h_lds_bytes<BM, BN>(), stream>>>(args);
      else
        gemm_w4h_kernel<BM, BN, IRIS_EPI_SILU_MUL, float, false><<<all, 256, w4h_lds_bytes<BM, BN>(), stream>>>(args);
      return check_launch("gemm_bf16");
    }
  }
  if (epilogue == kEpiQkRope) {
    // one tile per workgroup: the next tile's loads in flight would spill the store's registers
    if constexpr (BM == 256 && BN == 256) {
      gemm_w4h_kernel<BM, BN, kEpiQkRope, bf16, false><<<all, 256, w4h_lds_bytes<BM, BN>(), stream>>>(args);
      return check_launch("gemm_bf16");
    }
  }
  if (epilogue != IRIS_EPI_NONE)
    return fail(IRIS_E_UNSUPPORTED, "gemm: the %dx%d tile has no such epilogue", BM, BN);
  const int cus = device_cus();
  if (c_dtype == IRIS_BF16)
    gemm_w4h_kernel<BM, BN, IRIS_EPI_NONE, bf16, true>
        <<<dim3(args.total_tiles < cus ? args.total_tiles : cus), 256, w4h_lds_bytes<BM, BN>(), stream>>>(args);
  else
    gemm_w4h_kernel<BM, BN, IRIS_EPI_NONE, float, false>
        <<<dim3(args.total_tiles), 256, w4h_lds_bytes<BM, BN>(), stream>>>(args);
  return check_launch("gemm_bf16");
}

struct TileShape {
  int bm, bn, bk, stages, wgm, wgn, parts;
  bool w4 = false;   // gemm_w4_kernel: four waves of 128 x 128, register-staged refills
  bool w4h = false;  // gemm_w4h_kernel: four waves on the 16 x 16 x 32 MFMA
  bool swiglu() const { return w4h ? (bn / 2) % 64 == 0 : (bn / wgn / 32) % 2 == 0; }
};
// BM x BN output tile, BK-deep K tiles in a ring of `stages`, wgm x wgn waves, the refill of a
// K tile spread over `parts` k-steps.
constexpr TileShape kTiles[] = {
    {256, 256, 64, 2, 2, 4, 1},  // 0
    {256, 256, 64, 2, 2, 4, 2},  // 1
    {256, 192, 64, 2, 4, 2, 1},  // 2
    {256, 192, 64, 2, 4, 2, 2},  // 3
    {192, 256, 64, 2, 2, 4, 1},  // 4
    {192, 256, 64, 2, 2, 4, 2},  // 5
    {128, 128, 64, 2, 2, 2, 1},  // 6: two workgroups per CU
    {256, 256, 32, 4, 2, 4, 1},  // 7
    {256, 256, 32, 4, 2, 4, 2},  // 8
    {256, 256, 64, 2, 2, 2, 1},  // 9: one wave per SIMD
    {256, 256, 64, 2, 2, 2, 2},  // 10
    {256, 256, 64, 2, 2, 2, 1, true},  // 11: gemm_w4_kernel
    {192, 256, 64, 2, 2, 2, 1, true},  // 12: gemm_w4_kernel, 96 x 128 per wave
    {288, 160, 64, 2, 2, 2, 1, false, true},  // 13: gemm_w4h_kernel, 144 x 80 per wave
    {256, 160, 64, 2, 2, 2, 1, false, true},  // 14: gemm_w4h_kernel, 128 x 80 per wave
    {128, 160, 64, 2, 2, 2, 1, false, true},  // 15: gemm_w4h_kernel, 64 x 80 per wave
    {256, 256, 64, 2, 2, 2, 1, false, true},  // 16: gemm_w4h_kernel, 128 x 128 per wave
    {192, 256, 64, 2, 2, 2, 1, false, true},  // 17: gemm_w4h_kernel, 96 x 128 per wave
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

template <int I>
int launch_index(GemmArgs& args, int c_dtype, int epilogue, hipStream_t stream) {
  constexpr TileShape t = kTiles[I];
  if constexpr (t.w4) {
    static_assert((t.bm == 256 || t.bm == 192) && t.bn == 256 && t.bk == 64, "gemm_w4_kernel tile");
    return launch_w4<t.bm>(args, c_dtype, epilogue, stream);
  } else if constexpr (t.w4h) {
    static_assert(t.bk == 64, "gemm_w4h_kernel tile");
    return launch_w4h<t.bm, t.bn>(args, c_dtype, epilogue, stream);
  } else {
    return launch_tile<t.bm, t.bn, t.bk, t.stages, t.wgm, t.wgn, t.parts>(args, c_dtype, epilogue, stream);
  }
}

// Tile shape: the candidate with the least estimated time, rounds of workgroups over the
// device's CUs (256 on MI355X; the last round costs as much as a full one) x tile area /
// relative per-CU rate.
// Plain, bias and SwiGLU outputs run on the four-wave tiles of the 16 x 16 x 32 MFMA. Their
// rates are per-CU throughputs measured in one round of the microbenchmark (six weight copies,
// one box), relative to the 32 x 32 x 16 four-wave 256 x 256 tile's 1.12: 256 x 256 (16) 1.17
// (SwiGLU 4352 x 11520 x 2560, 765 tiles: 200 against 213 us on tile 11), 288 x 160 (13) 1.15,
// 256 x 160 (14) 1.12, 192 x 256 (17) 1.05, 128 x 160 (15) 0.88.
// The SiLU epilogue runs on the eight-wave tiles of the 32 x 32 x 16 MFMA, ranked inside the
// denoise step (alternating runs of the whole step on one box): 256 x 256 with direct-to-LDS
// refills (1) 1.09, 192 x 256 (5) 0.98, 256 x 192 (3) 0.96, 128 x 128 at two workgroups per CU
// (6) 0.9. The four-wave 32 x 32 x 16 tiles (11, 12) are the q|k|v store's and forced-only;
// so are the eight-wave 4-stage ring of 32-deep K tiles (8; 282 us on SwiGLU, although 8%
// faster than tile 1 in back-to-back runs), and four waves with direct-to-LDS refills (9, 10;
// 280-290 us).
struct Candidate {
  int tile, per_cu;
  double rate;
};
constexpr Candidate kCandidates[] = {{16, 1, 1.17}, {13, 1, 1.15}, {14, 1, 1.12}, {17, 1, 1.05}, {15, 1, 0.88},
                                     {1, 1, 1.09},  {5, 1, 0.98},  {3, 1, 0.96},  {6, 2, 0.9}};
constexpr int kSquare = 0;  // the 256 x 256 candidate of the 16 x 16 x 32 family
// The q|k|v projection's store (one tile row per thread, two heads per row) runs on the
// 256 x 256 tile of the family of the plain GEMM, so its outputs are bitwise those of
// iris_gemm_bf16 followed by iris_qkv_prepare.
constexpr int kQkRopeTile = 16;
static_assert(kCandidates[kSquare].tile == 16, "256 x 256 16 x 16 x 32 tile");

// Estimated time of one launch with candidate c (arbitrary units: tile area / rate per round).
double launch_cost(const Candidate& c, const int* m, int groups, int n, int cus) {
  const TileShape t = kTiles[c.tile];
  long tiles = 0;
  for (int i = 0; i < groups; ++i) tiles += static_cast<long>((m[i] + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
  const long slots = static_cast<long>(cus) * c.per_cu;
  return static_cast<double>((tiles + slots - 1) / slots) * t.bm * t.bn * c.per_cu / c.rate;
}

// The MFMA shape of a launch depends on the epilogue only, never on the row count or the width:
// the 16 x 16 x 32 MFMA sums 32 products per instruction, the 32 x 32 x 16 one 16, so the two
// families round differently, and a row's result must not depend on the other rows of the
// batch (nor a column's on where a column split falls).
bool mfma16_family(int epilogue) { return epilogue == IRIS_EPI_NONE || epilogue == IRIS_EPI_SILU_MUL; }

bool allowed(const Candidate& c, int epilogue) {
  const TileShape t = kTiles[c.tile];
  return t.w4h == mfma16_family(epilogue) && !(epilogue == IRIS_EPI_SILU_MUL && !t.swiglu()) &&
         !(epilogue == IRIS_EPI_SILU && (t.w4 || t.w4h));
}

int pick_tile(const int* m, int groups, int n, int epilogue, int forced, double* cost_out = nullptr) {
  if (forced >= 0) return forced;
  const int cus = device_cus();
  int best = -1;
  double best_cost = 0.0;
  for (const Candidate& c : kCandidates) {
    if (!allowed(c, epilogue)) continue;
    const double cost = launch_cost(c, m, groups, n, cus);
    if (best < 0 || cost < best_cost) best = c.tile, best_cost = cost;
  }
  if (cost_out) *cost_out = best_cost;
  return best;
}

// Column split: when the last round of 256 x 256 tiles would leave many CUs idle, the first n1
// columns run as whole rounds of 256 x 256 tiles (tile 16) and the rest with their own tile
// choice, e.g. SwiGLU 4352 x 13696: 765 tiles (3 rounds) + 207 tiles of 192 x 256 (one round)
// instead of 918 tiles in 4 rounds; both parts in one launch of gemm_w4h_pair_kernel where it
// has the pair of tiles, else two launches. The second part is charged a fixed cost (~3 us, the
// gap between two launches). Measured in the denoise step (on the 32 x 32 x 16 tiles, two
// launches then): 0.09 ms per step faster (the round model overstates the gain: the tiles of a
// partly filled last round run faster than those of a full one). n1 = 0: no split.
struct SplitPlan {
  int n1 = 0, tile1 = 16, tile2 = 16;
};
SplitPlan plan_split(const int* m, int groups, int n, int epilogue, int forced) {
  SplitPlan plan;
  const Candidate& sq = kCandidates[kSquare];
  // the first part always runs on the 256 x 256 tile: no split for an epilogue it does not have
  if (forced >= 0 || !allowed(sq, epilogue)) return plan;
  double whole = 0.0;
  plan.tile1 = pick_tile(m, groups, n, epilogue, -1, &whole);
  const int cus = device_cus();
  const double extra_launch = 65536.0 / sq.rate * 0.05;
  double best = 0.98 * whole;  // a split must win by 2%
  for (int c = 1; c * 256 < n; ++c) {
    const int n1 = 256 * c, n2 = n - n1;
    const double part1 = launch_cost(sq, m, groups, n1, cus);
    double part2 = 0.0;
    const int t2 = pick_tile(m, groups, n2, epilogue, -1, &part2);
    const double cost = part1 + part2 + extra_launch;
    // on equal estimates the widest first part: more of the work on the 256 x 256 tile
    if (cost <= best) best = cost, plan.n1 = n1, plan.tile1 = sq.tile, plan.tile2 = t2;
  }
  return plan;
}

// per thread: a forced tile never changes another thread's launches
thread_local int g_forced_tile = -1;

// Launch arguments of one GEMM over output columns [0, n) of operands already offset to the
// part's first column, on tile shape `tile`.
int make_args(GemmArgs& args, int groups, const void* const* a, const void* const* b, const float* const* bias,
              void* const* c, const int* m, int n, int k, long lda, long ldb, long ldc, int epilogue, int tile,
              const QkRope* qk) {
  args = GemmArgs{};
  if (qk) args.qk = *qk;
  args.ngroups = groups;
  args.n = n;
  args.k = k;
  args.lda = lda;
  args.ldb = ldb;
  args.ldc = ldc;
  const TileShape shape = kTiles[tile];
  const int bm = shape.bm;
  const int bn = shape.bn;
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
  IRIS_REQUIRE(epilogue != IRIS_EPI_SILU_MUL || shape.swiglu(), "gemm: tile %dx%d has no SwiGLU epilogue", bm, bn);
  return IRIS_OK;
}

// The (tile, epilogue) pairs gemm_w4h_pair_kernel is instantiated for, BF16 output: SwiGLU's
// two column parts (256 x 256, then 192 x 256) and the q|k|v store beside the gate columns
// (256 x 256, then 288 x 160).
bool has_pair(int tile1, int epi1, int tile2, int epi2) {
  return (tile1 == 16 && epi1 == IRIS_EPI_SILU_MUL && tile2 == 17 && epi2 == IRIS_EPI_SILU_MUL) ||
         (tile1 == kQkRopeTile && epi1 == kEpiQkRope && tile2 == 13 && epi2 == IRIS_EPI_NONE);
}

int launch_pair(const GemmArgs& a1, int epi1, const GemmArgs& a2, hipStream_t stream) {
  const dim3 grid(((a1.total_tiles + 7) & ~7) + a2.total_tiles);
  constexpr unsigned lds = w4h_lds_bytes<256, 256>();  // the larger ring of both pairs
  static_assert(lds >= w4h_lds_bytes<192, 256>() && lds >= w4h_lds_bytes<288, 160>(), "pair ring");
  if (epi1 == IRIS_EPI_SILU_MUL)
    gemm_w4h_pair_kernel<256, 256, IRIS_EPI_SILU_MUL, 192, 256, IRIS_EPI_SILU_MUL><<<grid, 256, lds, stream>>>(a1, a2);
  else
    gemm_w4h_pair_kernel<256, 256, kEpiQkRope, 288, 160, IRIS_EPI_NONE><<<grid, 256, lds, stream>>>(a1, a2);
  return check_launch("gemm_bf16 (two GEMMs)");
}

int launch_args(GemmArgs& args, int c_dtype, int epilogue, int tile, hipStream_t stream);

// One launch over output columns [0, n) of operands already offset to the part's first column.
int gemm_part(int groups, const void* const* a, const void* const* b, const float* const* bias, void* const* c,
              const int* m, int c_dtype, int n, int k, long lda, long ldb, long ldc, int epilogue, int tile,
              hipStream_t stream, const QkRope* qk = nullptr) {
  GemmArgs args;
  const int rc = make_args(args, groups, a, b, bias, c, m, n, k, lda, ldb, ldc, epilogue, tile, qk);
  if (rc != IRIS_OK) return rc;
  if (args.total_tiles == 0) return IRIS_OK;
  return launch_args(args, c_dtype, epilogue, tile, stream);
}

int launch_args(GemmArgs& args, int c_dtype, int epilogue, int tile, hipStream_t stream) {
  static_assert(kNumTiles == 18, "one case per tile shape");
  switch (tile) {
#define IRIS_TILE_CASE(I) \
  case I:                 \
    return launch_index<I>(args, c_dtype, epilogue, stream);
    IRIS_TILE_CASE(0)
    IRIS_TILE_CASE(1)
    IRIS_TILE_CASE(2)
    IRIS_TILE_CASE(3)
    IRIS_TILE_CASE(4)
    IRIS_TILE_CASE(5)
    IRIS_TILE_CASE(6)
    IRIS_TILE_CASE(7)
    IRIS_TILE_CASE(8)
    IRIS_TILE_CASE(9)
    IRIS_TILE_CASE(10)
    IRIS_TILE_CASE(11)
    IRIS_TILE_CASE(12)
    IRIS_TILE_CASE(13)
    IRIS_TILE_CASE(14)
    IRIS_TILE_CASE(15)
    IRIS_TILE_CASE(16)
    IRIS_TILE_CASE(17)
#undef IRIS_TILE_CASE
    default:
      return fail(IRIS_E_INVALID, "gemm: no tile shape %d", tile);
  }
}

// Two GEMMs, in one launch when has_pair allows it and both have tiles, else one after the
// other; the results are the same either way (one MFMA family, every tile sums k in order).
int launch_two(GemmArgs& a1, int tile1, int epi1, GemmArgs& a2, int tile2, int epi2, int c_dtype,
               hipStream_t stream) {
  if (c_dtype == IRIS_BF16 && has_pair(tile1, epi1, tile2, epi2) && a1.total_tiles > 0 && a2.total_tiles > 0)
    return launch_pair(a1, epi1, a2, stream);
  if (a1.total_tiles > 0) {
    const int rc = launch_args(a1, c_dtype, epi1, tile1, stream);
    if (rc != IRIS_OK) return rc;
  }
  return a2.total_tiles > 0 ? launch_args(a2, c_dtype, epi2, tile2, stream) : IRIS_OK;
}

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_gemm_bf16_grouped(int groups, const void* const* a, const void* const* b,
                                      const float* const* bias, void* const* c, const int* m, int c_dtype, int n,
                                      int k, long lda, long ldb, long ldc, int epilogue, hipStream_t stream) {
  IRIS_REQUIRE(groups == 1 || groups == 2, "gemm: 1 or 2 groups");
  IRIS_REQUIRE(c_dtype == IRIS_F32 || c_dtype == IRIS_BF16, "gemm: unknown output dtype");
  IRIS_REQUIRE(epilogue == IRIS_EPI_NONE || epilogue == IRIS_EPI_SILU_MUL || epilogue == IRIS_EPI_SILU,
               "gemm: unknown epilogue");
  IRIS_REQUIRE(n > 0 && k > 0 && k % kBK == 0, "gemm: need n > 0 and k %% 64 == 0 (got n=%d k=%d)", n, k);
  IRIS_REQUIRE(n % 4 == 0, "gemm: n %% 4 == 0 required (got %d)", n);
  IRIS_REQUIRE(epilogue != IRIS_EPI_SILU_MUL || n % 64 == 0, "gemm: the SwiGLU epilogue needs n %% 64 == 0");
  IRIS_REQUIRE(lda >= k && ldb >= k && lda % 8 == 0 && ldb % 8 == 0, "gemm: lda/ldb must be >= k and multiples of 8");
  IRIS_REQUIRE(ldc >= (epilogue == IRIS_EPI_SILU_MUL ? n / 2 : n) && ldc % 4 == 0, "gemm: bad ldc");
  for (int i = 0; i < groups; ++i) {
    IRIS_REQUIRE(m[i] >= 0, "gemm: negative m");
    IRIS_REQUIRE(m[i] == 0 || (a[i] && b[i] && c[i]), "gemm: null pointer");
    IRIS_REQUIRE(!a[i] || (aligned(a[i], 16) && aligned(b[i], 16) && aligned(c[i], 16)),
                 "gemm: operands must be 16-byte aligned");
    IRIS_REQUIRE(!bias || !bias[i] || epilogue != IRIS_EPI_SILU_MUL, "gemm: bias is not supported with SwiGLU");
  }
  // byte offsets and buffer sizes are 32-bit ints (elements x 2): below 2 GiB per operand
  IRIS_REQUIRE(static_cast<long>(n) * ldb < (1L << 30), "gemm: weight above 2 GiB (32-bit byte offsets)");
  for (int i = 0; i < groups; ++i)
    IRIS_REQUIRE(static_cast<long>(m[i]) * lda < (1L << 30), "gemm: activation above 2 GiB (32-bit byte offsets)");
  const SplitPlan plan = plan_split(m, groups, n, epilogue, g_forced_tile);
  if (plan.n1 == 0)
    return gemm_part(groups, a, b, bias, c, m, c_dtype, n, k, lda, ldb, ldc, epilogue,
                     pick_tile(m, groups, n, epilogue, g_forced_tile), stream);
  // columns [0, n1) and [n1, n): weight rows, bias entries and output columns of the second part
  // start at n1 (n1 / 2 output columns for SwiGLU); one launch for both where a pair kernel exists
  GemmArgs a1, a2;
  int rc = make_args(a1, groups, a, b, bias, c, m, plan.n1, k, lda, ldb, ldc, epilogue, plan.tile1, nullptr);
  if (rc != IRIS_OK) return rc;
  const void* b2[2];
  const float* bias2[2];
  void* c2[2];
  const long out_col = epilogue == IRIS_EPI_SILU_MUL ? plan.n1 / 2 : plan.n1;
  const size_t out_size = c_dtype == IRIS_BF16 ? 2 : 4;
  for (int i = 0; i < groups; ++i) {
    b2[i] = b[i] ? static_cast<const bf16*>(b[i]) + static_cast<long>(plan.n1) * ldb : nullptr;
    bias2[i] = bias && bias[i] ? bias[i] + plan.n1 : nullptr;
    c2[i] = c[i] ? static_cast<char*>(c[i]) + out_col * out_size : nullptr;
  }
  rc = make_args(a2, groups, a, b2, bias ? bias2 : nullptr, c2, m, n - plan.n1, k, lda, ldb, ldc, epilogue, plan.tile2,
                 nullptr);
  if (rc != IRIS_OK) return rc;
  return launch_two(a1, plan.tile1, epilogue, a2, plan.tile2, epilogue, c_dtype, stream);
}

extern "C" int iris_gemm_bf16_qk_rope(int groups, const void* const* a, const void* const* b, void* const* c,
                                      const int* m, int n, int k, long lda, long ldb, long ldc,
                                      const float* const* q_weight, const float* const* k_weight,
                                      const int* rows_per_batch, const int* dst_offset, const float* cos_table,
                                      const float* sin_table, long table_rows, void* q, void* k_out, int heads,
                                      int kv_heads, long n_dst, void* vt, long n_vt, float eps, hipStream_t stream) {
  IRIS_REQUIRE(groups == 1 || groups == 2, "gemm_qk_rope: 1 or 2 groups");
  IRIS_REQUIRE(heads > 0 && kv_heads > 0 && n % 128 == 0 && n >= (heads + kv_heads) * 128,
               "gemm_qk_rope: n (%d) must be whole 128-wide heads covering the %d Q and %d K heads", n, heads,
               kv_heads);
  IRIS_REQUIRE(k > 0 && k % kBK == 0, "gemm_qk_rope: need k > 0 and k %% 64 == 0 (got %d)", k);
  IRIS_REQUIRE(lda >= k && ldb >= k && lda % 8 == 0 && ldb % 8 == 0, "gemm_qk_rope: lda/ldb must be >= k and multiples of 8");
  IRIS_REQUIRE(ldc >= n && ldc % 8 == 0, "gemm_qk_rope: ldc must be >= n and a multiple of 8");
  IRIS_REQUIRE(q && k_out && cos_table && sin_table && q_weight && k_weight && rows_per_batch && dst_offset,
               "gemm_qk_rope: null pointer");
  IRIS_REQUIRE(aligned(q, 16) && aligned(k_out, 16) && aligned(cos_table, 16) && aligned(sin_table, 16),
               "gemm_qk_rope: q, k and the rotary tables must be 16-byte aligned");
  IRIS_REQUIRE(n_dst > 0 && n_dst < (1L << 30) && table_rows > 0, "gemm_qk_rope: bad n_dst / table_rows");
  for (int i = 0; i < groups; ++i) {
    IRIS_REQUIRE(m[i] >= 0, "gemm_qk_rope: negative m");
    if (m[i] == 0) continue;
    IRIS_REQUIRE(a[i] && b[i] && c[i] && q_weight[i] && k_weight[i], "gemm_qk_rope: null pointer");
    IRIS_REQUIRE(aligned(a[i], 16) && aligned(b[i], 16) && aligned(c[i], 16) && aligned(q_weight[i], 16) &&
                     aligned(k_weight[i], 16),
                 "gemm_qk_rope: operands and gains must be 16-byte aligned");
    IRIS_REQUIRE(rows_per_batch[i] > 0 && m[i] % rows_per_batch[i] == 0,
                 "gemm_qk_rope: m (%d) must be whole batch items of %d rows", m[i], rows_per_batch[i]);
    IRIS_REQUIRE(dst_offset[i] >= 0 && dst_offset[i] + static_cast<long>(rows_per_batch[i]) <= n_dst &&
                     dst_offset[i] + static_cast<long>(rows_per_batch[i]) <= table_rows,
                 "gemm_qk_rope: positions %d..%d outside q/k (%ld) or the rotary table (%ld)", dst_offset[i],
                 dst_offset[i] + rows_per_batch[i] - 1, n_dst, table_rows);
    IRIS_REQUIRE(static_cast<long>(m[i]) * lda < (1L << 30), "gemm_qk_rope: activation above 2 GiB (32-bit byte offsets)");
  }
  IRIS_REQUIRE(static_cast<long>(n) * ldb < (1L << 30), "gemm_qk_rope: weight above 2 GiB (32-bit byte offsets)");
  const int n_qkv = (heads + 2 * kv_heads) * 128;  // Q, K and V heads; any columns after them are plain
  if (vt) {
    // the kv_heads V heads go to vt (and no other column: the plain columns go to c)
    IRIS_REQUIRE(n >= n_qkv, "gemm_qk_rope: with vt, n (%d) must cover the %d Q, %d K and %d V heads of 128 columns",
                 n, heads, kv_heads, kv_heads);
    IRIS_REQUIRE(aligned(vt, 16) && n_vt > 0 && n_vt % 64 == 0 && n_vt < (1L << 30),
                 "gemm_qk_rope: vt must be 16-byte aligned with n_vt a positive multiple of 64");
    for (int i = 0; i < groups; ++i)
      IRIS_REQUIRE(m[i] == 0 || (rows_per_batch[i] % 256 == 0 && dst_offset[i] % 16 == 0 &&
                                 dst_offset[i] + static_cast<long>(rows_per_batch[i]) <= n_vt),
                   "gemm_qk_rope: the V^T store needs rows_per_batch %% 256 == 0, dst_offset %% 16 == 0 and "
                   "positions inside vt (group %d: %d rows at %d, n_vt %ld)",
                   i, rows_per_batch[i], dst_offset[i], n_vt);
  }
  const int g1 = groups > 1 ? 1 : 0;
  QkRope qk{};
  qk.q = static_cast<bf16*>(q);
  qk.k = static_cast<bf16*>(k_out);
  qk.cos = cos_table;
  qk.sin = sin_table;
  qk.q_weight0 = q_weight[0];
  qk.q_weight1 = q_weight[g1];
  qk.k_weight0 = k_weight[0];
  qk.k_weight1 = k_weight[g1];
  qk.rows_per_batch0 = rows_per_batch[0];
  qk.rows_per_batch1 = rows_per_batch[g1];
  qk.dst_offset0 = dst_offset[0];
  qk.dst_offset1 = dst_offset[g1];
  qk.n_dst = static_cast<int>(n_dst);
  qk.heads = heads;
  qk.kv_heads = kv_heads;
  qk.eps = eps;
  qk.vt = static_cast<bf16*>(vt);
  qk.n_vt = static_cast<int>(n_vt);
  if (n <= n_qkv)
    return gemm_part(groups, a, b, nullptr, c, m, IRIS_BF16, n, k, lda, ldb, ldc, kEpiQkRope, kQkRopeTile, stream, &qk);
  // the columns after the V heads (the gate columns of a q | k | v | gate weight) are a plain
  // product into c beside the store, in the same launch where a pair kernel exists
  GemmArgs a1, a2;
  int rc = make_args(a1, groups, a, b, nullptr, c, m, n_qkv, k, lda, ldb, ldc, kEpiQkRope, kQkRopeTile, &qk);
  if (rc != IRIS_OK) return rc;
  const void* b2[2];
  void* c2[2];
  for (int i = 0; i < groups; ++i) {
    b2[i] = b[i] ? static_cast<const bf16*>(b[i]) + static_cast<long>(n_qkv) * ldb : nullptr;
    c2[i] = c[i] ? static_cast<bf16*>(c[i]) + n_qkv : nullptr;
  }
  const int tile2 = pick_tile(m, groups, n - n_qkv, IRIS_EPI_NONE, g_forced_tile);
  rc = make_args(a2, groups, a, b2, nullptr, c2, m, n - n_qkv, k, lda, ldb, ldc, IRIS_EPI_NONE, tile2, nullptr);
  if (rc != IRIS_OK) return rc;
  return launch_two(a1, kQkRopeTile, kEpiQkRope, a2, tile2, IRIS_EPI_NONE, IRIS_BF16, stream);
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

// Tuning hook: force a tile shape (an index into kTiles, -1: automatic).
extern "C" int iris_gemm_force_tile(int tile) {
  IRIS_REQUIRE(tile >= -1 && tile < kNumTiles, "gemm_force_tile: tile in -1..%d", kNumTiles - 1);
  g_forced_tile = tile;
  return IRIS_OK;
}
