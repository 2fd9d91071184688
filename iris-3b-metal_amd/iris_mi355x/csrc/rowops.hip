// Row-wise bandwidth kernels of the trunk: RMSNorm + adaLN modulate, post-norm gated
// residual (optionally fused with the next RMSNorm + modulate), per-head qk-RMSNorm + 2-D
// RoPE, the V-head transpose, and small row utilities.
//
// Layout: one 64-lane wave per D-wide row; lane l owns the 8-element chunks l, l + 64, ...
// (16-byte BF16 / 32-byte FP32 accesses, 1 KB or 2 KB contiguous per wave instruction), and
// the row stays in registers between the statistics pass and the output pass, so HBM sees
// each byte once.
#include "iris_common.hpp"

namespace iris {
namespace {

constexpr int kRowsPerBlock = 4;  // one row per wave, 4 waves per 256-thread workgroup

// 8 elements of a row held in their storage type (BF16 rows take half the registers of FP32
// ones, which keeps more waves, and more loads in flight, per CU).
template <typename T>
struct Chunk8;
template <>
struct Chunk8<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ float operator[](int e) const { return to_f32(v[e]); }
};
template <>
struct Chunk8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float operator[](int e) const { return e < 4 ? a[e] : b[e - 4]; }
};

// NC = 8-element chunks each lane holds (width <= NC * 512). A wave issues its row's loads
// first, reduces, and reads the per-column FP32 coefficients chunk by chunk in the output pass,
// so they need no registers across the row. SHARED (the four rows of a workgroup share one
// batch index): the workgroup combines weight * (1 + scale) and copies shift into LDS once while
// its rows' loads are in flight, and the waves read them there (the same products as the
// per-wave form, so the results are identical) instead of three L2 reads per chunk.
template <int NC, typename TI, typename TO, bool SHARED>
__global__ __launch_bounds__(256) void rms_norm_modulate_kernel(const TI* __restrict__ x, TO* __restrict__ out,
                                                                const float* __restrict__ weight,
                                                                const float* __restrict__ shift,
                                                                const float* __restrict__ scale, long rows,
                                                                long rows_per_batch, int width, long mod_stride,
                                                                float eps) {
  const long row0 = static_cast<long>(blockIdx.x) * 4;
  const long row = row0 + (threadIdx.x >> 6);
  if (!SHARED && row >= rows) return;
  const bool active = row < rows;  // (SHARED: every wave takes part in the LDS fill)
  const int lane = threadIdx.x & 63;
  const int nc = width >> 3;
  Chunk8<TI> v[NC];
  if (active) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int j = lane + i * kWave;
      if (j < nc) v[i].load(x + row * width + 8 * j);
    }
  }
  extern __shared__ __attribute__((aligned(16))) float mcoef[];  // [w (1 + scale) | shift], width each
  if constexpr (SHARED) {
    const long bs = row0 / rows_per_batch;
    for (int c = 4 * static_cast<int>(threadIdx.x); c < width; c += 4 * 256) {
      const f32x4 wv = load4(weight + c), s1 = load4(scale + bs * mod_stride + c);
      *reinterpret_cast<f32x4*>(mcoef + c) = wv * (1.0f + s1);
      *reinterpret_cast<f32x4*>(mcoef + width + c) = load4(shift + bs * mod_stride + c);
    }
    __syncthreads();
    if (!active) return;
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
  }
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(width) + eps);
  const long b = row / rows_per_batch;
  TO* o = out + row * width;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc) {
      float m[8], c0[8], y[8];
      if constexpr (SHARED) {
        load8(mcoef + 8 * j, m);
        load8(mcoef + width + 8 * j, c0);
      } else {
        float w[8], s1[8];
        load8(weight + 8 * j, w);
        load8(scale + b * mod_stride + 8 * j, s1);
        load8(shift + b * mod_stride + 8 * j, c0);
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = w[e] * (1.0f + s1[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (v[i][e] * r) * m[e] + c0[e];
      store8(o + 8 * j, y);
    }
  }
}

// residual[r] += gate * rmsnorm(branch[r]) * weight; with next_out, also
// next_out[r] = rmsnorm(residual[r]) * next_weight * (1 + next_scale) + next_shift from the
// updated row still in registers (the next branch's input norm, without re-reading the row).
// Coefficients (gate * weight, and next_weight * (1 + next_scale), next_shift) are held per
// wave as in rms_norm_modulate_kernel.
// One launch serves up to two groups of rows with their own tensors (the image and text streams
// of a dual-stream block): workgroups [0, blocks0) take group 0, the rest group 1.
struct GatedGroup {
  float* residual;
  const void* branch;
  const float* weight;
  const float* gate;
  long rows, rows_per_batch, mod_stride;
  const float* next_weight;
  const float* next_shift;
  const float* next_scale;
  long next_mod_stride;
  void* next_out;
};
struct GatedArgs {
  GatedGroup g[2];
  long blocks0;
  int width;
  float eps;
};

// SHARED (with the next norm; the four rows of a workgroup share one batch index): the
// workgroup combines the coefficient vectors once into LDS (gate * weight, next_weight *
// (1 + next_scale) and next_shift, the same products as the per-wave form, so results are
// identical) while its rows' loads are in flight, and each wave reads them there: no L2 round
// trip per 8-column chunk on the way out (-10% per call), and a quarter of the L2 reads.
// At width 2560 with BF16 branches that form fits five waves per SIMD (96 VGPRs): 5120 rows in
// flight, so a 4352-row launch needs one round instead of two.
template <int NC, typename TB, typename TO, bool SHARED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(SHARED && NC == 5 && sizeof(TB) == 2 ? 5 : 1)))
void gated_residual_kernel(GatedArgs a) {
  const bool second = blockIdx.x >= a.blocks0;
  const GatedGroup& gg = second ? a.g[1] : a.g[0];
  float* __restrict__ residual = gg.residual;
  const TB* __restrict__ branch = static_cast<const TB*>(gg.branch);
  const float* __restrict__ weight = gg.weight;
  const float* __restrict__ gate = gg.gate;
  const long rows = gg.rows, rows_per_batch = gg.rows_per_batch, mod_stride = gg.mod_stride;
  const float* __restrict__ next_weight = gg.next_weight;
  const float* __restrict__ next_shift = gg.next_shift;
  const float* __restrict__ next_scale = gg.next_scale;
  const long next_mod_stride = gg.next_mod_stride;
  TO* __restrict__ next_out = static_cast<TO*>(gg.next_out);
  const int width = a.width;
  const float eps = a.eps;
  const long row0 = (static_cast<long>(blockIdx.x) - (second ? a.blocks0 : 0)) * 4;
  const long row = row0 + (threadIdx.x >> 6);
  if (!SHARED && row >= rows) return;
  const bool active = row < rows;  // (SHARED: every wave takes part in the LDS fill)
  const int lane = threadIdx.x & 63;
  const int nc = width >> 3;
  Chunk8<TB> v[NC];
  float x[NC][8];
  float* res = residual + row * width;
  if (active) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int j = lane + i * kWave;
      if (j < nc) {
        v[i].load(branch + row * width + 8 * j);
        load8(res + 8 * j, x[i]);
      }
    }
  }
  extern __shared__ __attribute__((aligned(16))) float coef[];  // [gw | nw | sh], width each
  if constexpr (SHARED) {
    const long bs = row0 / rows_per_batch;
    for (int c = 4 * static_cast<int>(threadIdx.x); c < width; c += 4 * 256) {
      const f32x4 gv = load4(gate + bs * mod_stride + c), wv = load4(weight + c);
      const f32x4 w2 = load4(next_weight + c), s1 = load4(next_scale + bs * next_mod_stride + c);
      *reinterpret_cast<f32x4*>(coef + c) = gv * wv;
      *reinterpret_cast<f32x4*>(coef + width + c) = w2 * (1.0f + s1);
      *reinterpret_cast<f32x4*>(coef + 2 * width + c) = load4(next_shift + bs * next_mod_stride + c);
    }
    __syncthreads();
    if (!active) return;
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
  }
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(width) + eps);
  const long b = row / rows_per_batch;
  float ss2 = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc) {
      float gw[8];
      if constexpr (SHARED) {
        load8(coef + 8 * j, gw);
      } else {
        float w[8], g[8];
        load8(weight + 8 * j, w);
        load8(gate + b * mod_stride + 8 * j, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) gw[e] = g[e] * w[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[i][e] += gw[e] * (v[i][e] * r);
        ss2 += x[i][e] * x[i][e];
      }
      store8(res + 8 * j, x[i]);
    }
  }
  if (next_out == nullptr) return;
  const float r2 = rsqrtf(wave_sum(ss2) / static_cast<float>(width) + eps);
  TO* o = next_out + row * width;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc) {
      float m[8], c0[8], y[8];
      if constexpr (SHARED) {
        load8(coef + width + 8 * j, m);
        load8(coef + 2 * width + 8 * j, c0);
      } else {
        float w2[8], s1[8];
        load8(next_weight + 8 * j, w2);
        load8(next_scale + b * next_mod_stride + 8 * j, s1);
        load8(next_shift + b * next_mod_stride + 8 * j, c0);
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = w2[e] * (1.0f + s1[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (x[i][e] * r2) * m[e] + c0[e];
      store8(o + 8 * j, y);
    }
  }
}

// 16 lanes per (token, head) row of 128 values; lane s owns elements [8s, 8s+8) = rotary
// pairs 4s..4s+3. A 16-lane group handles up to kQkRows heads of one token (all loads issued
// before the first reduction, the token's rotary row read once), 16 groups per workgroup.
constexpr int kQkRows = 4;

// Workgroup `block` of batch `b` (16 groups of 16 lanes).
template <typename TI, typename TO>
__device__ __forceinline__ void qk_norm_rope_block(const TI* __restrict__ src, TO* __restrict__ dst,
                                                   const float* __restrict__ weight,
                                                   const float* __restrict__ cos_table,
                                                   const float* __restrict__ sin_table, long n_src, long n_dst,
                                                   int heads, long dst_offset, long row_stride, long col_offset,
                                                   float eps, long block, long b) {
  // group = (token, up to kQkRows consecutive heads): the rotary row is read once per group
  const int head_groups = (heads + kQkRows - 1) / kQkRows;
  const long grp = block * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (grp >= n_src * head_groups) return;  // whole 16-lane groups leave together
  const long token = grp / head_groups;
  const int head0 = static_cast<int>(grp - token * head_groups) * kQkRows;
  const TI* xr = src + (b * n_src + token) * row_stride + col_offset + 8 * sub;
  float a[kQkRows][8];
#pragma unroll
  for (int k = 0; k < kQkRows; ++k) load8(xr + min(head0 + k, heads - 1) * 128, a[k]);
  float w[8];
  load8(weight + 8 * sub, w);
  const long out_token = dst_offset + token;
  const f32x4 c = load4(cos_table + out_token * 64 + 4 * sub);
  const f32x4 s = load4(sin_table + out_token * 64 + 4 * sub);
#pragma unroll
  for (int k = 0; k < kQkRows; ++k) {
    const int head = head0 + k;
    float y[8];
    head_norm_rope(a[k], w, c, s, eps, y);  // all 16 lanes; clamped heads are not stored
    if (head >= heads) continue;
    store8(dst + ((b * heads + head) * n_dst + out_token) * 128 + 8 * sub, y);
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const TI* __restrict__ src, TO* __restrict__ dst,
                                                           const float* __restrict__ weight,
                                                           const float* __restrict__ cos_table,
                                                           const float* __restrict__ sin_table, long n_src,
                                                           long n_dst, int heads, long dst_offset, long row_stride,
                                                           long col_offset, float eps) {
  qk_norm_rope_block<TI, TO>(src, dst, weight, cos_table, sin_table, n_src, n_dst, heads, dst_offset, row_stride,
                             col_offset, eps, blockIdx.x, blockIdx.y);
}

// Transpose the V heads into dst[b, h, d, position]: one workgroup per (64 output positions
// aligned to 64, head, batch). Position P holds token vt_slot(P) - dst_offset; LDS rows are
// padded by 8 elements (272 bytes) so the column reads of the second phase spread over banks.
// Workgroup (position block `pblock`, head, batch b); every thread of the workgroup takes part.
__device__ __forceinline__ void v_heads_t_block(const bf16* __restrict__ src, bf16* __restrict__ dst, long n_src,
                                                long n_dst, int heads, long dst_offset, long row_stride,
                                                long col_offset, long pblock, int head, long b,
                                                bf16 (*tile)[136]) {
  const long p0 = (dst_offset / 64 + pblock) * 64;  // first output position of the block
  const long t0 = p0 - dst_offset;                   // token of position p0 (may be < 0)
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;  // 64 token slots x 16 chunks of 8
    const int slot = idx >> 4;
    const int c = idx & 15;
    const long tok = t0 + slot;
    bf16x8 v = {};
    if (tok >= 0 && tok < n_src)
      v = *reinterpret_cast<const bf16x8*>(src + (b * n_src + tok) * row_stride + col_offset + head * 128 + 8 * c);
    *reinterpret_cast<bf16x8*>(&tile[slot][8 * c]) = v;
  }
  __syncthreads();
  bf16* out = dst + (b * heads + head) * 128 * n_dst + p0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;  // 128 dims x 8 chunks of 8 positions
    const int d = idx >> 3;
    const int c = idx & 7;
    bf16x8 v;
    int valid = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int slot = vt_slot(8 * c + e);
      v[e] = tile[slot][d];
      valid += (t0 + slot >= 0 && t0 + slot < n_src) ? 1 : 0;
    }
    if (valid == 0) continue;
    bf16* o = out + static_cast<long>(d) * n_dst + 8 * c;
    if (valid == 8 && (n_dst & 7) == 0) {
      *reinterpret_cast<bf16x8*>(o) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int slot = vt_slot(8 * c + e);
        if (t0 + slot >= 0 && t0 + slot < n_src) o[e] = v[e];
      }
    }
  }
}

__global__ __launch_bounds__(256) void v_heads_t_kernel(const bf16* __restrict__ src, bf16* __restrict__ dst,
                                                        long n_src, long n_dst, int heads, long dst_offset,
                                                        long row_stride, long col_offset) {
  __shared__ bf16 tile[64][136];
  v_heads_t_block(src, dst, n_src, n_dst, heads, dst_offset, row_stride, col_offset, blockIdx.x, blockIdx.y,
                  blockIdx.z, tile);
}

// Q and K per-head RMSNorm + RoPE and the V^T transpose of one projection in one launch:
// workgroups [0, q_blocks) run qk_norm_rope on the Q heads, [q_blocks, q_blocks + k_blocks) on
// the K heads, the rest transpose the V heads (position block major, then head).
struct QkvPrepareArgs {
  const bf16* src;
  bf16 *q, *k, *vt;
  const float *q_weight, *k_weight, *cos_table, *sin_table;
  long n_src, n_dst, n_vt, dst_offset, row_stride, q_col, k_col, v_col;
  int heads, kv_heads;
  long q_blocks, k_blocks, v_pos_blocks;
  float eps;
};

__global__ __launch_bounds__(256) void qkv_prepare_kernel(QkvPrepareArgs a) {
  __shared__ bf16 tile[64][136];
  const long bx = blockIdx.x;
  const long b = blockIdx.y;
  if (bx < a.q_blocks) {
    qk_norm_rope_block<bf16, bf16>(a.src, a.q, a.q_weight, a.cos_table, a.sin_table, a.n_src, a.n_dst, a.heads,
                                   a.dst_offset, a.row_stride, a.q_col, a.eps, bx, b);
  } else if (bx < a.q_blocks + a.k_blocks) {
    qk_norm_rope_block<bf16, bf16>(a.src, a.k, a.k_weight, a.cos_table, a.sin_table, a.n_src, a.n_dst, a.kv_heads,
                                   a.dst_offset, a.row_stride, a.k_col, a.eps, bx - a.q_blocks, b);
  } else {
    const long v = bx - a.q_blocks - a.k_blocks;
    v_heads_t_block(a.src, a.vt, a.n_src, a.n_vt, a.kv_heads, a.dst_offset, a.row_stride, a.v_col,
                    v % a.v_pos_blocks, static_cast<int>(v / a.v_pos_blocks), b, tile);
  }
}

template <typename TO>
__global__ __launch_bounds__(256) void silu_add_rows_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                            long rows, long rows_per_batch, int width,
                                                            TO* __restrict__ out) {
  const long i4 = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long nv = static_cast<long>(width) >> 2;
  if (i4 >= rows * nv) return;
  const long row = i4 / nv;
  const long col = (i4 - row * nv) * 4;
  const f32x4 a = load4(x + row * width + col);
  const f32x4 b = load4(t + (row / rows_per_batch) * width + col);
  f32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = silu(a[e] + b[e]);
  store4(out + row * width + col, y);
}

__global__ __launch_bounds__(256) void copy_rows_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                        long rows, int width, long src_batch_rows,
                                                        long src_row_offset, long dst_batch_rows,
                                                        long dst_row_offset) {
  const long i4 = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long nv = static_cast<long>(width) >> 2;
  if (i4 >= rows * nv) return;
  const long b = blockIdx.y;
  const long row = i4 / nv;
  const long col = (i4 - row * nv) * 4;
  store4(dst + (b * dst_batch_rows + dst_row_offset + row) * width + col,
         load4(src + (b * src_batch_rows + src_row_offset + row) * width + col));
}

// residual[r] += branch[r] (when a branch is given, stored back), then
// out[r] = rmsnorm(residual[r]) * weight (+ add_rows[r % add_period]): the pre-norm residual
// step of the text adapter's blocks, fused with the next input norm, or its final norm plus
// the position table.
template <int NC, typename TB, typename TO>
__global__ __launch_bounds__(256) void residual_norm_kernel(float* __restrict__ residual, const TB* __restrict__ branch,
                                                            const float* __restrict__ weight,
                                                            const float* __restrict__ add_rows, long add_period,
                                                            long rows, int width, float eps, TO* __restrict__ out) {
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nc = width >> 3;
  float* res = residual + row * width;
  float x[NC][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc) {
      load8(res + 8 * j, x[i]);
      if (branch) {
        float v[8];
        load8(branch + row * width + 8 * j, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[i][e] += v[e];
        store8(res + 8 * j, x[i]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
    }
  }
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(width) + eps);
  TO* o = out + row * width;
  const float* add = add_rows ? add_rows + (row % add_period) * width : nullptr;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int j = lane + i * kWave;
    if (j < nc) {
      float w[8], y[8];
      load8(weight + 8 * j, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (x[i][e] * r) * w[e];
      if (add) {
        float a[8];
        load8(add + 8 * j, a);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] += a[e];
      }
      store8(o + 8 * j, y);
    }
  }
}

template <int NC, bool SHARED>
void launch_rms_modulate(dim3 grid, size_t lds, hipStream_t stream, const void* x, int x_dtype, void* out,
                         int out_dtype, const float* weight, const float* shift, const float* scale, long rows,
                         long rows_per_batch, int width, long mod_stride, float eps) {
  if (x_dtype == IRIS_F32 && out_dtype == IRIS_BF16)
    rms_norm_modulate_kernel<NC, float, bf16, SHARED><<<grid, 256, lds, stream>>>(
        (const float*)x, (bf16*)out, weight, shift, scale, rows, rows_per_batch, width, mod_stride, eps);
  else if (x_dtype == IRIS_F32 && out_dtype == IRIS_F32)
    rms_norm_modulate_kernel<NC, float, float, SHARED><<<grid, 256, lds, stream>>>(
        (const float*)x, (float*)out, weight, shift, scale, rows, rows_per_batch, width, mod_stride, eps);
  else if (x_dtype == IRIS_BF16 && out_dtype == IRIS_BF16)
    rms_norm_modulate_kernel<NC, bf16, bf16, SHARED><<<grid, 256, lds, stream>>>(
        (const bf16*)x, (bf16*)out, weight, shift, scale, rows, rows_per_batch, width, mod_stride, eps);
  else
    rms_norm_modulate_kernel<NC, bf16, float, SHARED><<<grid, 256, lds, stream>>>(
        (const bf16*)x, (float*)out, weight, shift, scale, rows, rows_per_batch, width, mod_stride, eps);
}

int nc_bucket(int width) {
  const int need = (width / 8 + kWave - 1) / kWave;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 3) return 3;
  if (need <= 5) return 5;
  if (need <= 8) return 8;
  return 16;
}

#define IRIS_NC_DISPATCH(NCV, ...)                          \
  switch (NCV) {                                            \
    case 1: { constexpr int NC = 1; __VA_ARGS__; } break;   \
    case 2: { constexpr int NC = 2; __VA_ARGS__; } break;   \
    case 3: { constexpr int NC = 3; __VA_ARGS__; } break;   \
    case 5: { constexpr int NC = 5; __VA_ARGS__; } break;   \
    case 8: { constexpr int NC = 8; __VA_ARGS__; } break;   \
    default: { constexpr int NC = 16; __VA_ARGS__; } break; \
  }

bool valid_dtype(int dt) { return dt == IRIS_F32 || dt == IRIS_BF16; }

template <int NC, typename TB>
void launch_gated(dim3 grid, hipStream_t stream, const GatedArgs& a, int out_dtype, bool shared) {
  if (shared) {  // (with the next norm only)
    const size_t lds = 3 * static_cast<size_t>(a.width) * sizeof(float);
    if (out_dtype == IRIS_F32)
      gated_residual_kernel<NC, TB, float, true><<<grid, 256, lds, stream>>>(a);
    else
      gated_residual_kernel<NC, TB, bf16, true><<<grid, 256, lds, stream>>>(a);
  } else {
    if (out_dtype == IRIS_F32)
      gated_residual_kernel<NC, TB, float, false><<<grid, 256, 0, stream>>>(a);
    else
      gated_residual_kernel<NC, TB, bf16, false><<<grid, 256, 0, stream>>>(a);
  }
}

int check_group(const GatedGroup& g) {
  IRIS_REQUIRE(g.rows >= 0 && g.rows_per_batch > 0, "gated_residual_rms_norm: bad row counts");
  IRIS_REQUIRE(g.mod_stride % 4 == 0 && aligned(g.gate, 16) && aligned(g.weight, 16),
               "gated_residual_rms_norm: gate rows must be 16-byte aligned");
  IRIS_REQUIRE(g.residual && g.branch && g.weight && g.gate, "gated_residual_rms_norm: null pointer");
  IRIS_REQUIRE(!g.next_out || (g.next_weight && g.next_shift && g.next_scale && g.next_mod_stride % 4 == 0 &&
                               aligned(g.next_weight, 16) && aligned(g.next_shift, 16) && aligned(g.next_scale, 16)),
               "gated_residual_rms_norm: the next norm needs 16-byte aligned FP32 gain and modulation rows");
  return IRIS_OK;
}

// groups: 1 or 2 entries of g; both with or both without the next norm.
int gated_launch(int groups, const GatedGroup* g, int branch_dtype, int width, float eps, int out_dtype,
                 hipStream_t stream) {
  IRIS_REQUIRE(valid_dtype(branch_dtype) && valid_dtype(out_dtype), "gated_residual_rms_norm: unknown dtype");
  IRIS_REQUIRE(width > 0 && width % 128 == 0 && width <= 8192,
               "gated_residual_rms_norm_ shape mismatch: width %% 128 == 0 and <= 8192 (got %d)", width);
  GatedArgs a{};
  long blocks = 0;
  for (int i = 0; i < groups; ++i) {
    const int rc = check_group(g[i]);
    if (rc) return rc;
    IRIS_REQUIRE((g[i].next_out == nullptr) == (g[0].next_out == nullptr),
                 "gated_residual_rms_norm: both groups with or both without the next norm");
    a.g[i] = g[i];
    const long b = (g[i].rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (i == 0) a.blocks0 = b;
    blocks += b;
  }
  if (groups == 1) a.g[1] = a.g[0];
  a.width = width;
  a.eps = eps;
  if (blocks == 0) return IRIS_OK;
  IRIS_REQUIRE(blocks < (1L << 31), "gated_residual_rms_norm: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks));
  // with the next norm, coefficients in LDS when every workgroup's four rows share a batch
  // index (without it the LDS fill and its barrier cost more than the one coefficient row saves)
  const bool next = g[0].next_out != nullptr;
  bool shared = next && 3L * width * sizeof(float) <= 48 * 1024;
  for (int i = 0; i < groups; ++i) shared = shared && g[i].rows_per_batch % kRowsPerBlock == 0;
  IRIS_NC_DISPATCH(nc_bucket(width), {
    if (branch_dtype == IRIS_BF16)
      launch_gated<NC, bf16>(grid, stream, a, out_dtype, shared);
    else
      launch_gated<NC, float>(grid, stream, a, out_dtype, shared);
  })
  return check_launch("gated_residual_rms_norm");
}

int gated_common(float* residual, const void* branch, int branch_dtype, const float* weight, const float* gate,
                 long rows, long rows_per_batch, int width, long mod_stride, float eps, const float* nw,
                 const float* nsh, const float* nsc, long nstride, void* next_out, int out_dtype,
                 hipStream_t stream) {
  const GatedGroup g{residual, branch, weight, gate, rows, rows_per_batch, mod_stride, nw, nsh, nsc, nstride, next_out};
  return gated_launch(1, &g, branch_dtype, width, eps, out_dtype, stream);
}

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_rms_norm_modulate(const void* x, int x_dtype, void* out, int out_dtype, const float* weight,
                                      const float* shift, const float* scale, long rows, long rows_per_batch,
                                      int width, long mod_stride, float eps, hipStream_t stream) {
  IRIS_REQUIRE(valid_dtype(x_dtype) && valid_dtype(out_dtype), "rms_norm_modulate: unknown dtype");
  IRIS_REQUIRE(width > 0 && width % 128 == 0 && width <= 8192,
               "rms_norm_modulate needs a contiguous input, width %% 128 == 0 and <= 8192 (got %d)", width);
  IRIS_REQUIRE(rows >= 0 && rows_per_batch > 0, "rms_norm_modulate: bad row counts");
  IRIS_REQUIRE(mod_stride % 4 == 0 && aligned(shift, 16) && aligned(scale, 16) && aligned(weight, 16),
               "rms_norm_modulate: modulation rows must be 16-byte aligned (mod_stride %% 4 == 0)");
  IRIS_REQUIRE(x && out && weight && shift && scale, "rms_norm_modulate: null pointer");
  if (rows == 0) return IRIS_OK;
  const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  // coefficients in LDS when every workgroup's four rows share a batch index
  const bool shared = rows_per_batch % kRowsPerBlock == 0 && 2L * width * sizeof(float) <= 32 * 1024;
  IRIS_NC_DISPATCH(nc_bucket(width), {
    if (shared)
      launch_rms_modulate<NC, true>(grid, 2 * width * sizeof(float), stream, x, x_dtype, out, out_dtype, weight,
                                    shift, scale, rows, rows_per_batch, width, mod_stride, eps);
    else
      launch_rms_modulate<NC, false>(grid, 0, stream, x, x_dtype, out, out_dtype, weight, shift, scale, rows,
                                     rows_per_batch, width, mod_stride, eps);
  })
  return check_launch("rms_norm_modulate");
}

extern "C" int iris_gated_residual_rms_norm(float* residual, const void* branch, int branch_dtype,
                                            const float* weight, const float* gate, long rows, long rows_per_batch,
                                            int width, long mod_stride, float eps, hipStream_t stream) {
  return gated_common(residual, branch, branch_dtype, weight, gate, rows, rows_per_batch, width, mod_stride, eps,
                      nullptr, nullptr, nullptr, 0, nullptr, IRIS_BF16, stream);
}

extern "C" int iris_gated_residual_norm_modulate(float* residual, const void* branch, int branch_dtype,
                                                 const float* weight, const float* gate, long rows,
                                                 long rows_per_batch, int width, long mod_stride, float eps,
                                                 const float* next_weight, const float* next_shift,
                                                 const float* next_scale, long next_mod_stride, void* next_out,
                                                 int next_out_dtype, hipStream_t stream) {
  IRIS_REQUIRE(next_out != nullptr, "gated_residual_norm_modulate: next_out is required");
  return gated_common(residual, branch, branch_dtype, weight, gate, rows, rows_per_batch, width, mod_stride, eps,
                      next_weight, next_shift, next_scale, next_mod_stride, next_out, next_out_dtype, stream);
}

extern "C" int iris_gated_residual_grouped(int groups, float* const* residual, const void* const* branch,
                                           int branch_dtype, const float* const* weight, const float* const* gate,
                                           const long* rows, const long* rows_per_batch, int width,
                                           const long* mod_stride, float eps, const float* const* next_weight,
                                           const float* const* next_shift, const float* const* next_scale,
                                           const long* next_mod_stride, void* const* next_out, int next_out_dtype,
                                           hipStream_t stream) {
  IRIS_REQUIRE(groups == 1 || groups == 2, "gated_residual_grouped: 1 or 2 groups");
  IRIS_REQUIRE(residual && branch && weight && gate && rows && rows_per_batch && mod_stride,
               "gated_residual_grouped: null array");
  const bool next = next_out != nullptr;
  IRIS_REQUIRE(!next || (next_weight && next_shift && next_scale && next_mod_stride),
               "gated_residual_grouped: the next norm's arrays are missing");
  GatedGroup g[2] = {};
  for (int i = 0; i < groups; ++i) {
    g[i] = GatedGroup{residual[i], branch[i], weight[i], gate[i], rows[i], rows_per_batch[i], mod_stride[i],
                      next ? next_weight[i] : nullptr, next ? next_shift[i] : nullptr, next ? next_scale[i] : nullptr,
                      next ? next_mod_stride[i] : 0, next ? next_out[i] : nullptr};
    IRIS_REQUIRE(!next || g[i].next_out, "gated_residual_grouped: next_out %d is null", i);
  }
  return gated_launch(groups, g, branch_dtype, width, eps, next ? next_out_dtype : IRIS_BF16, stream);
}

extern "C" int iris_qk_norm_rope(const void* src, int src_dtype, void* dst, int dst_dtype, const float* weight,
                                 const float* cos_table, const float* sin_table, long table_rows, int batch,
                                 long n_src, long n_dst, int heads, long dst_offset, long row_stride,
                                 long col_offset, float eps, hipStream_t stream) {
  IRIS_REQUIRE(valid_dtype(src_dtype) && valid_dtype(dst_dtype), "qk_norm_rope: unknown dtype");
  IRIS_REQUIRE(heads > 0 && col_offset >= 0 && dst_offset >= 0, "heads must be positive and offsets nonnegative");
  IRIS_REQUIRE(batch >= 0 && batch <= 65535 && n_src >= 0, "qk_norm_rope: bad sizes");
  IRIS_REQUIRE(col_offset + heads * 128L <= row_stride,
               "qk_norm_rope needs a contiguous [B, N, W] input holding the heads");
  IRIS_REQUIRE(dst_offset + n_src <= table_rows && dst_offset + n_src <= n_dst,
               "qk_norm_rope rotary tables or output do not cover the written rows");
  IRIS_REQUIRE(row_stride % 8 == 0 && col_offset % 8 == 0, "qk_norm_rope: rows must be 16-byte aligned");
  IRIS_REQUIRE(src && dst && weight && cos_table && sin_table, "qk_norm_rope: null pointer");
  if (batch == 0 || n_src == 0) return IRIS_OK;
  const long groups = n_src * ((heads + kQkRows - 1) / kQkRows);  // (token, head group) pairs
  const dim3 grid(static_cast<unsigned>((groups + 15) / 16), static_cast<unsigned>(batch));
#define IRIS_QK_LAUNCH(TI, TO)                                                                                   \
  qk_norm_rope_kernel<TI, TO><<<grid, 256, 0, stream>>>((const TI*)src, (TO*)dst, weight, cos_table, sin_table, \
                                                        n_src, n_dst, heads, dst_offset, row_stride, col_offset, \
                                                        eps)
  if (src_dtype == IRIS_BF16 && dst_dtype == IRIS_BF16)
    IRIS_QK_LAUNCH(bf16, bf16);
  else if (src_dtype == IRIS_BF16)
    IRIS_QK_LAUNCH(bf16, float);
  else if (dst_dtype == IRIS_BF16)
    IRIS_QK_LAUNCH(float, bf16);
  else
    IRIS_QK_LAUNCH(float, float);
#undef IRIS_QK_LAUNCH
  return check_launch("qk_norm_rope");
}

extern "C" int iris_v_heads_t(const void* src, void* dst, int batch, long n_src, long n_dst, int heads,
                              long dst_offset, long row_stride, long col_offset, hipStream_t stream) {
  IRIS_REQUIRE(heads > 0 && heads <= 65535 && batch >= 0 && batch <= 65535 && n_src >= 0,
               "v_heads_t: bad sizes");
  IRIS_REQUIRE(col_offset >= 0 && col_offset + heads * 128L <= row_stride && row_stride % 8 == 0 &&
                   col_offset % 8 == 0,
               "v_heads_t: heads must lie in 16-byte aligned rows of the projection");
  IRIS_REQUIRE(dst_offset >= 0 && dst_offset + n_src <= n_dst, "v_heads_t: output does not cover the rows");
  IRIS_REQUIRE(n_dst % 64 == 0, "v_heads_t: the V^T rows must be a multiple of 64 positions");
  IRIS_REQUIRE(src && dst, "v_heads_t: null pointer");
  if (batch == 0 || n_src == 0) return IRIS_OK;
  const long first = dst_offset / 64, last = (dst_offset + n_src + 63) / 64;
  const dim3 grid(static_cast<unsigned>(last - first), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
  v_heads_t_kernel<<<grid, 256, 0, stream>>>((const bf16*)src, (bf16*)dst, n_src, n_dst, heads, dst_offset,
                                             row_stride, col_offset);
  return check_launch("v_heads_t");
}

extern "C" int iris_qkv_prepare(const void* src, void* q, void* k, void* vt, const float* q_weight,
                                const float* k_weight, const float* cos_table, const float* sin_table,
                                long table_rows, int batch, long n_src, long n_dst, long n_vt, int heads,
                                int kv_heads, long dst_offset, long row_stride, long q_col, long k_col, long v_col,
                                float eps, hipStream_t stream) {
  IRIS_REQUIRE(heads > 0 && kv_heads > 0 && kv_heads <= 65535, "qkv_prepare: bad head counts");
  IRIS_REQUIRE(batch >= 0 && batch <= 65535 && n_src >= 0, "qkv_prepare: bad sizes");
  IRIS_REQUIRE(q_col >= 0 && k_col >= 0 && v_col >= 0 && q_col + heads * 128L <= row_stride &&
                   k_col + kv_heads * 128L <= row_stride && v_col + kv_heads * 128L <= row_stride,
               "qkv_prepare needs a contiguous [B, N, W] projection holding the Q, K and V heads");
  IRIS_REQUIRE(row_stride % 8 == 0 && q_col % 8 == 0 && k_col % 8 == 0 && v_col % 8 == 0,
               "qkv_prepare: rows must be 16-byte aligned");
  IRIS_REQUIRE(dst_offset >= 0 && dst_offset + n_src <= table_rows && dst_offset + n_src <= n_dst &&
                   dst_offset + n_src <= n_vt,
               "qkv_prepare: rotary tables or outputs do not cover the written rows");
  IRIS_REQUIRE(n_vt % 64 == 0, "qkv_prepare: the V^T rows must be a multiple of 64 positions");
  IRIS_REQUIRE(src && q && k && vt && q_weight && k_weight && cos_table && sin_table, "qkv_prepare: null pointer");
  if (batch == 0 || n_src == 0) return IRIS_OK;
  QkvPrepareArgs a{static_cast<const bf16*>(src), static_cast<bf16*>(q), static_cast<bf16*>(k),
                   static_cast<bf16*>(vt), q_weight, k_weight, cos_table, sin_table, n_src, n_dst, n_vt,
                   dst_offset, row_stride, q_col, k_col, v_col, heads, kv_heads, 0, 0, 0, eps};
  a.q_blocks = (n_src * ((heads + kQkRows - 1) / kQkRows) + 15) / 16;
  a.k_blocks = (n_src * ((kv_heads + kQkRows - 1) / kQkRows) + 15) / 16;
  a.v_pos_blocks = (dst_offset + n_src + 63) / 64 - dst_offset / 64;
  const long blocks = a.q_blocks + a.k_blocks + a.v_pos_blocks * kv_heads;
  IRIS_REQUIRE(blocks < (1L << 31), "qkv_prepare: too many rows");
  qkv_prepare_kernel<<<dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(batch)), 256, 0, stream>>>(a);
  return check_launch("qkv_prepare");
}

extern "C" int iris_silu_add_rows(const float* x, const float* t, long rows, long rows_per_batch, int width,
                                  void* out, int out_dtype, hipStream_t stream) {
  IRIS_REQUIRE(valid_dtype(out_dtype), "silu_add_rows: unknown dtype");
  IRIS_REQUIRE(width > 0 && width % 4 == 0 && rows >= 0 && rows_per_batch > 0, "silu_add_rows: bad sizes");
  IRIS_REQUIRE(x && t && out, "silu_add_rows: null pointer");
  if (rows == 0) return IRIS_OK;
  const long n4 = rows * (width / 4);
  const dim3 grid(static_cast<unsigned>((n4 + 255) / 256));
  if (out_dtype == IRIS_BF16)
    silu_add_rows_kernel<bf16><<<grid, 256, 0, stream>>>(x, t, rows, rows_per_batch, width, (bf16*)out);
  else
    silu_add_rows_kernel<float><<<grid, 256, 0, stream>>>(x, t, rows, rows_per_batch, width, (float*)out);
  return check_launch("silu_add_rows");
}

extern "C" int iris_copy_rows(const float* src, float* dst, int batch, long rows, int width, long src_batch_rows,
                              long src_row_offset, long dst_batch_rows, long dst_row_offset, hipStream_t stream) {
  IRIS_REQUIRE(width > 0 && width % 4 == 0 && rows >= 0 && batch >= 0 && batch <= 65535, "copy_rows: bad sizes");
  IRIS_REQUIRE(src_row_offset >= 0 && dst_row_offset >= 0 && src_row_offset + rows <= src_batch_rows &&
                   dst_row_offset + rows <= dst_batch_rows,
               "copy_rows: row block outside its batch");
  IRIS_REQUIRE(src && dst, "copy_rows: null pointer");
  if (rows == 0 || batch == 0) return IRIS_OK;
  const long n4 = rows * (width / 4);
  const dim3 grid(static_cast<unsigned>((n4 + 255) / 256), static_cast<unsigned>(batch));
  copy_rows_kernel<<<grid, 256, 0, stream>>>(src, dst, rows, width, src_batch_rows, src_row_offset, dst_batch_rows,
                                             dst_row_offset);
  return check_launch("copy_rows");
}

extern "C" int iris_residual_rms_norm(float* residual, const void* branch, int branch_dtype, const float* weight,
                                      const float* add_rows, long add_period, long rows, int width, float eps,
                                      void* out, int out_dtype, hipStream_t stream) {
  IRIS_REQUIRE(valid_dtype(branch_dtype) && valid_dtype(out_dtype), "residual_rms_norm: unknown dtype");
  IRIS_REQUIRE(width > 0 && width % 8 == 0 && width <= 8192, "residual_rms_norm: width %% 8 == 0 and <= 8192 (got %d)",
               width);
  IRIS_REQUIRE(rows >= 0 && (!add_rows || add_period > 0), "residual_rms_norm: bad row counts");
  IRIS_REQUIRE(residual && weight && out, "residual_rms_norm: null pointer");
  IRIS_REQUIRE(aligned(residual, 16) && aligned(weight, 16) && aligned(out, 16) && (!branch || aligned(branch, 16)) &&
                   (!add_rows || aligned(add_rows, 16)),
               "residual_rms_norm: rows must be 16-byte aligned");
  IRIS_REQUIRE(out != residual && (!branch || (branch != residual && branch != out)),
               "residual_rms_norm: out and branch must not alias the residual");
  if (rows == 0) return IRIS_OK;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  IRIS_NC_DISPATCH(nc_bucket(width), {
    if (branch_dtype == IRIS_BF16 && out_dtype == IRIS_BF16)
      residual_norm_kernel<NC, bf16, bf16><<<grid, 256, 0, stream>>>(residual, (const bf16*)branch, weight, add_rows,
                                                                     add_period, rows, width, eps, (bf16*)out);
    else if (branch_dtype == IRIS_BF16)
      residual_norm_kernel<NC, bf16, float><<<grid, 256, 0, stream>>>(residual, (const bf16*)branch, weight, add_rows,
                                                                      add_period, rows, width, eps, (float*)out);
    else if (out_dtype == IRIS_BF16)
      residual_norm_kernel<NC, float, bf16><<<grid, 256, 0, stream>>>(residual, (const float*)branch, weight,
                                                                      add_rows, add_period, rows, width, eps,
                                                                      (bf16*)out);
    else
      residual_norm_kernel<NC, float, float><<<grid, 256, 0, stream>>>(residual, (const float*)branch, weight,
                                                                       add_rows, add_period, rows, width, eps,
                                                                       (float*)out);
  })
  return check_launch("residual_rms_norm");
}
