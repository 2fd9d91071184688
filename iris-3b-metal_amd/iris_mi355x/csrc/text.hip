// Kernels of the layer-wise text adapter (src/iris3b/nn/embeddings.py:110-141, 209-266) that
// the GEMM, row and flash-attention kernels do not cover: the self-attention of each text
// token across its encoder layers (a sequence of a dozen states per token, so one wave per
// (token, head) with the whole sequence in LDS), and the learned pool over those layers.
#include "iris_common.hpp"

#include <algorithm>

namespace iris {
namespace {

constexpr int kMaxSeq = 16;    // encoder layers per token
constexpr int kMaxHeadDim = 128;
constexpr int kMaxWavesPerBlock = 4;
constexpr int kLdsBudget = 64 * 1024;  // bytes of LDS per workgroup the launch may ask for

// LDS floats of one wave: q, k, v of L tokens of d values, and the L x L probabilities.
__host__ __device__ constexpr int layer_attention_floats(int L, int d) { return 3 * L * d + L * L; }

// One wave per (sequence s, head h): q, k, v rows of the L tokens of sequence s are columns
// h*d, D + h*d, 2D + h*d of qkv rows s*L .. s*L + L - 1 (D = heads * d). out = softmax(q k^T *
// scale) v in FP32 from BF16 inputs, stored BF16 at out rows s*L + i, columns h*d. A block holds
// blockDim.x / 64 waves, each with its own LDS slice.
__global__ __launch_bounds__(64 * kMaxWavesPerBlock) void layer_attention_kernel(const bf16* __restrict__ qkv,
                                                                              bf16* __restrict__ out, long seqs,
                                                                              int L, int heads, int d, float scale) {
  extern __shared__ float smem[];
  const int wv = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const long item = static_cast<long>(blockIdx.x) * (blockDim.x >> 6) + wv;
  const bool active = item < seqs * heads;  // every wave reaches the barriers
  float* sq = smem + wv * layer_attention_floats(L, d);
  float* sk = sq + L * d;
  float* sv = sk + L * d;
  float* sp = sv + L * d;
  const long s = active ? item / heads : 0;
  const int h = active ? static_cast<int>(item % heads) : 0;
  const int D = heads * d;
  if (active) {
    for (int e = lane; e < L * d; e += kWave) {
      const int i = e / d, c = e - i * d;
      const bf16* row = qkv + (s * L + i) * 3L * D + h * d + c;
      sq[e] = to_f32(row[0]);
      sk[e] = to_f32(row[D]);
      sv[e] = to_f32(row[2 * D]);
    }
  }
  __syncthreads();
  if (active) {
    for (int e = lane; e < L * L; e += kWave) {
      const int i = e / L, j = e - i * L;
      float acc = 0.0f;
      for (int c = 0; c < d; ++c) acc += sq[i * d + c] * sk[j * d + c];
      sp[e] = acc * scale;
    }
  }
  __syncthreads();
  if (active && lane < L) {
    float* pr = sp + lane * L;
    float m = -INFINITY;
    for (int j = 0; j < L; ++j) m = fmaxf(m, pr[j]);
    float sum = 0.0f;
    for (int j = 0; j < L; ++j) {
      const float p = expf(pr[j] - m);
      pr[j] = p;
      sum += p;
    }
    const float inv = 1.0f / sum;
    for (int j = 0; j < L; ++j) pr[j] *= inv;
  }
  __syncthreads();
  if (active) {
    for (int e = lane; e < L * d; e += kWave) {
      const int i = e / d, c = e - i * d;
      float acc = 0.0f;
      for (int j = 0; j < L; ++j) acc += sp[i * L + j] * sv[j * d + c];
      out[(s * L + i) * static_cast<long>(D) + h * d + c] = from_f32<bf16>(acc);
    }
  }
}

// 0/1 key bytes [batch, n_pad] from a [batch, >= n] mask of 1-, 4- or 8-byte elements (bool /
// uint8, int32, float32, int64: nonzero = keep, as mask.bool()); positions n .. n_pad - 1 are 0.
__global__ __launch_bounds__(256) void key_mask_kernel(const void* __restrict__ mask, int kind, long ld, int batch,
                                                       int n, int n_pad, unsigned char* __restrict__ out) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<long>(batch) * n_pad) return;
  const long b = i / n_pad;
  const int j = static_cast<int>(i - b * n_pad);
  bool keep = false;
  if (j < n) {
    const long at = b * ld + j;
    switch (kind) {
      case 0:
        keep = static_cast<const unsigned char*>(mask)[at] != 0;
        break;
      case 1:
        keep = static_cast<const int*>(mask)[at] != 0;
        break;
      case 2:
        keep = static_cast<const float*>(mask)[at] != 0.0f;
        break;
      default:
        keep = static_cast<const long long*>(mask)[at] != 0;
        break;
    }
  }
  out[i] = keep ? 1 : 0;
}

// out[r, c] = sum_l weight[l] * (h + branch)[r*L + l, c] + bias, in layer order (nn.Linear(L, 1)
// over the layer axis, after the last block's residual add); four columns per thread.
template <typename TO>
__global__ __launch_bounds__(256) void layer_pool_kernel(const float* __restrict__ h, const bf16* __restrict__ branch,
                                                         const float* __restrict__ weight,
                                                         const float* __restrict__ bias, long rows, int L, int width,
                                                         TO* __restrict__ out) {
  const long i4 = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long nv = width >> 2;
  if (i4 >= rows * nv) return;
  const long r = i4 / nv;
  const int c = static_cast<int>(i4 - r * nv) * 4;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int l = 0; l < L; ++l) {
    f32x4 v = load4(h + (r * L + l) * width + c);
    if (branch) {
      const f32x4 bv = load4(branch + (r * L + l) * width + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += bv[e];
    }
    const float wl = weight[l];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += wl * v[e];
  }
  const float b = bias ? bias[0] : 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] += b;
  store4(out + r * width + c, acc);
}

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_layer_attention(const void* qkv, void* out, long seqs, int seq_len, int heads, int head_dim,
                                    float scale, hipStream_t stream) {
  IRIS_REQUIRE(seqs >= 0 && seq_len > 0 && seq_len <= kMaxSeq && heads > 0 && head_dim > 0 &&
                   head_dim <= kMaxHeadDim,
               "layer_attention: sequences of 1..%d tokens with heads of at most %d (got %d, %d)", kMaxSeq,
               kMaxHeadDim, seq_len, head_dim);
  IRIS_REQUIRE(qkv && out && qkv != out, "layer_attention: bad pointers");
  if (seqs == 0) return IRIS_OK;
  const long items = seqs * heads;
  const size_t per_wave = sizeof(float) * layer_attention_floats(seq_len, head_dim);  // <= 25.6 KB
  const int waves = static_cast<int>(std::min<size_t>(kMaxWavesPerBlock, kLdsBudget / per_wave));
  IRIS_REQUIRE((items + waves - 1) / waves < (1L << 31), "layer_attention: grid too large");
  const dim3 grid(static_cast<unsigned>((items + waves - 1) / waves));
  layer_attention_kernel<<<grid, 64 * waves, per_wave * waves, stream>>>(static_cast<const bf16*>(qkv),
                                                                         static_cast<bf16*>(out), seqs, seq_len,
                                                                         heads, head_dim, scale);
  return check_launch("layer_attention");
}

extern "C" int iris_text_key_mask(const void* mask, int elem_kind, long ld, int batch, long n, long n_pad, void* out,
                                  hipStream_t stream) {
  IRIS_REQUIRE(elem_kind >= 0 && elem_kind <= 3, "text_key_mask: element kind 0 (1 byte), 1 (int32), 2 (float32), 3 (int64)");
  IRIS_REQUIRE(batch >= 0 && n > 0 && n_pad >= n && n_pad % 64 == 0 && n_pad < (1L << 24) && ld >= n,
               "text_key_mask: bad shape");
  IRIS_REQUIRE(mask && out && aligned(out, 4), "text_key_mask: bad pointers");
  if (batch == 0) return IRIS_OK;
  const long total = batch * n_pad;
  key_mask_kernel<<<dim3(static_cast<unsigned>((total + 255) / 256)), 256, 0, stream>>>(
      mask, elem_kind, ld, batch, static_cast<int>(n), static_cast<int>(n_pad), static_cast<unsigned char*>(out));
  return check_launch("text_key_mask");
}

extern "C" int iris_layer_pool(const float* h, const void* branch, const float* weight, const float* bias, long rows,
                               int layers, int width, void* out, int out_dtype, hipStream_t stream) {
  IRIS_REQUIRE(rows >= 0 && layers > 0 && width > 0 && width % 4 == 0, "layer_pool: bad shape");
  IRIS_REQUIRE(out_dtype == IRIS_F32 || out_dtype == IRIS_BF16, "layer_pool: unknown output dtype");
  IRIS_REQUIRE(h && weight && out && aligned(h, 16) && aligned(out, 8) && (!branch || aligned(branch, 8)),
               "layer_pool: bad pointers");
  if (rows == 0) return IRIS_OK;
  const long n = rows * (width / 4);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (out_dtype == IRIS_F32)
    layer_pool_kernel<float><<<grid, 256, 0, stream>>>(h, static_cast<const bf16*>(branch), weight, bias, rows, layers,
                                                       width, static_cast<float*>(out));
  else
    layer_pool_kernel<bf16><<<grid, 256, 0, stream>>>(h, static_cast<const bf16*>(branch), weight, bias, rows, layers,
                                                      width, static_cast<bf16*>(out));
  return check_launch("layer_pool");
}
