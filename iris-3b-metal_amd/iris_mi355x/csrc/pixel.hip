// Pixel-stage bandwidth kernels: patchify + pixel embedding, the per-pixel RMSNorm, the
// post-modulated PiT tail (norm, 16 -> 64 -> 16 exact-GELU MLP, both modulated residual
// adds, next block's norm) and the 16 -> 3 head with unpatchify. One thread per pixel and
// FP32 math (BF16 only where the value is stored), except the MLP's two products, which run
// on BF16 MFMA at the reference's BF16 rounding points.
#include <algorithm>

#include "iris_common.hpp"

namespace iris {
namespace {

constexpr int kPix = 16;      // pixel channel width of the PiT stage
constexpr int kHidden = 64;   // PiT MLP hidden width

// C input channels: 3 (RGB) or 4 (the depth fine-tune's RGB + zero channel).
template <typename TP, int C>
__global__ __launch_bounds__(256) void patchify_embed_kernel(
    const float* __restrict__ x, int batch, int height, int width, int patch, bf16* __restrict__ patches,
    long patch_stride, const float* __restrict__ pix_w, const float* __restrict__ pix_b, const float* __restrict__ pos_x,
    const float* __restrict__ pos_y, const float* __restrict__ norm_w, float eps, TP* __restrict__ pixels,
    bf16* __restrict__ normed) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long hw = static_cast<long>(height) * width;
  if (idx >= batch * hw) return;
  const int px_x = static_cast<int>(idx % width);
  const int px_y = static_cast<int>((idx / width) % height);
  const long b = idx / hw;
  float v[C];
#pragma unroll
  for (int c = 0; c < C; ++c) v[c] = x[(b * C + c) * hw + static_cast<long>(px_y) * width + px_x];
  const int wp = width / patch;
  const long n_patches = static_cast<long>(height / patch) * wp;
  const long l = static_cast<long>(px_y / patch) * wp + px_x / patch;
  const int in_patch = (px_y % patch) * patch + (px_x % patch);
  const int pp = patch * patch;
  bf16* prow = patches + (b * n_patches + l) * patch_stride + in_patch;
#pragma unroll
  for (int c = 0; c < C; ++c) prow[c * pp] = from_f32<bf16>(v[c]);

  float e[kPix];
  float ss = 0.0f;
#pragma unroll
  for (int ch = 0; ch < kPix; ++ch) {
    float acc = v[0] * pix_w[ch * C + 0];
#pragma unroll
    for (int c = 1; c < C; ++c) acc += v[c] * pix_w[ch * C + c];
    acc += pix_b[ch];
    acc += ch < kPix / 2 ? pos_x[px_x * (kPix / 2) + ch] : pos_y[px_y * (kPix / 2) + ch - kPix / 2];
    e[ch] = acc;
    ss += acc * acc;
  }
  const long q = (b * n_patches + l) * pp + in_patch;
  store8(pixels + q * kPix, e);
  store8(pixels + q * kPix + 8, e + 8);
  const float r = rsqrtf(ss / kPix + eps);
  float h[kPix];
#pragma unroll
  for (int ch = 0; ch < kPix; ++ch) h[ch] = (e[ch] * r) * norm_w[ch];
  store8(normed + q * kPix, h);
  store8(normed + q * kPix + 8, h + 8);
}

template <typename TP>
__global__ __launch_bounds__(256) void pixel_rms_norm_kernel(const TP* __restrict__ pixels, bf16* __restrict__ out,
                                                             const float* __restrict__ weight, long n_pixels,
                                                             float eps) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n_pixels) return;
  float v[kPix];
  load8(pixels + idx * kPix, v);
  load8(pixels + idx * kPix + 8, v + 8);
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kPix; ++c) ss += v[c] * v[c];
  const float r = rsqrtf(ss / kPix + eps);
#pragma unroll
  for (int c = 0; c < kPix; ++c) v[c] = (v[c] * r) * weight[c];
  store8(out + idx * kPix, v);
  store8(out + idx * kPix + 8, v + 8);
}

#include "gelu_bf16_table.inc"

constexpr unsigned kGeluLo = kGeluLowExponent << 7;  // |bits| of the first table argument
constexpr unsigned kGeluN = kGeluPerSign;

// GELU of a pre-activation rounded to BF16, itself rounded to BF16 (the pixel MLP's two
// rounding points, src/iris_metal/kernels.py:273-274), from the correctly rounded table of the
// BF16 arguments 2^-16 <= |a| < 256 held in LDS. Below that range a Phi(a) lies within half an
// ulp of a / 2, above it GELU(a) is a (a > 0) or underflows to 0; all three cases agree with
// the correctly rounded exact-erf GELU for every finite BF16 argument. A NaN passes through,
// -inf gives 0.
__device__ __forceinline__ bf16 gelu_bf16(float a, const unsigned short* tab) {
  const bf16 ab = static_cast<bf16>(a);
  const unsigned u = __builtin_bit_cast(unsigned short, ab);
  const unsigned t = (u & 0x7fffu) - kGeluLo;  // wraps for |a| < 2^-16
  const unsigned short tv = tab[min(t, kGeluN - 1) + (u >> 15) * kGeluN];
  const float af = static_cast<float>(ab);
  const float outside = static_cast<int>(t) < 0 ? 0.5f * af : (af <= 0.0f ? 0.0f : af);
  return t < kGeluN ? __builtin_bit_cast(bf16, tv) : static_cast<bf16>(outside);
}

// The table-only GELU of two pre-activations, packed as a BF16 pair; `worst` collects the
// largest table offset seen (an offset >= kGeluN marks an argument outside the table, whose
// entry here is a clamped stand-in that the caller must replace).
__device__ __forceinline__ unsigned gelu2_table(float a0, float a1, const unsigned short* tab, unsigned& worst) {
  const unsigned pk = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a0, a1}, bf16x2));
  const unsigned t0 = (pk & 0x7fffu) - kGeluLo;
  const unsigned t1 = ((pk >> 16) & 0x7fffu) - kGeluLo;
  worst = max(worst, max(t0, t1));
  const unsigned v0 = tab[min(t0, kGeluN - 1) + ((pk >> 15) & 1u) * kGeluN];
  const unsigned v1 = tab[min(t1, kGeluN - 1) + (pk >> 31) * kGeluN];
  return v0 | (v1 << 16);
}

// Sum of a lane's value and its partner's (lane ^ 32); the same bits on both, as the sum commutes.
__device__ __forceinline__ float pair_sum(float v) { return v + __shfl_xor(v, 32); }

// One lane's share of a pixel as it comes from memory: 8 stream channels, 8 branch channels
// and the 4 x 8 modulation values of those channels.
template <typename TP>
struct PixelShare {
  TP x[8];
  bf16x8 br, s1, t1, s2, t2;
};

template <typename TP>
__device__ __forceinline__ void load_share(PixelShare<TP>& d, const TP* pixels, const bf16* branch, const bf16* mods,
                                           long idx, int c0) {
  if constexpr (sizeof(TP) == 4) {
    *reinterpret_cast<f32x4*>(d.x) = *reinterpret_cast<const f32x4*>(pixels + idx * kPix + c0);
    *reinterpret_cast<f32x4*>(d.x + 4) = *reinterpret_cast<const f32x4*>(pixels + idx * kPix + c0 + 4);
  } else {
    *reinterpret_cast<bf16x8*>(d.x) = *reinterpret_cast<const bf16x8*>(pixels + idx * kPix + c0);
  }
  d.br = *reinterpret_cast<const bf16x8*>(branch + idx * kPix + c0);
  const bf16* m = mods + idx * 4 * kPix + c0;
  d.s1 = *reinterpret_cast<const bf16x8*>(m);
  d.t1 = *reinterpret_cast<const bf16x8*>(m + kPix);
  d.s2 = *reinterpret_cast<const bf16x8*>(m + 2 * kPix);
  d.t2 = *reinterpret_cast<const bf16x8*>(m + 3 * kPix);
}

// The PiT tail on BF16 MFMA. A wave takes 32 pixels per step; lane l owns pixel l % 32 and
// channels 8 (l / 32) .. 8 (l / 32) + 7, which is both the B-operand layout of
// v_mfma_f32_32x32x16_bf16 (column l % 32, k = 8 (l / 32) + m) and, for the 16 output rows
// of the second product, the accumulator layout once the rows are put in channel order
// chan(i) (bits 2 and 3 of the row index swapped). Per step:
//   x += branch (1 + scale1) + shift1; h = bf16(rmsnorm(x) * norm_w)        (FP32, two lanes)
//   A^T[64 hidden, 32 px] = W1 h^T + b1                                      (2 MFMAs, K = 16)
//   G = gelu_bf16(A^T), in place: the accumulator registers 8 jj .. 8 jj + 7 of hidden block
//       blk are exactly a B operand over hidden units 32 blk + 16 jj + 8 (m / 4) + 4 (l / 32)
//       + m % 4, and W2's columns are gathered in that order
//   Y^T[16 ch, 32 px] = W2 G + b2                                            (4 MFMAs, K = 64)
//   x += Y (1 + scale2) + shift2; pixels = x; next_input = bf16(rmsnorm(x) * next_w)
// The weights (FP32 in memory) are rounded to BF16 as operands; sums accumulate in FP32. The
// RMS sums add each lane's 8 squares in channel order and then the two halves. G comes from
// the table alone unless some argument of the step lies outside it (|a| < 2^-16 or >= 256,
// rare for O(1) activations): then the wave recomputes the step's G with the full rule. The
// next step's inputs are loaded while the current one computes; lanes past the last pixel
// load the last pixel and store nothing.
template <typename TP>
__global__ __launch_bounds__(256) void pixel_mlp_kernel(
    TP* __restrict__ pixels, const bf16* __restrict__ branch, const bf16* __restrict__ mods,
    const float* __restrict__ norm_w, const float* __restrict__ fc1_w, const float* __restrict__ fc1_b,
    const float* __restrict__ fc2_w, const float* __restrict__ fc2_b, const float* __restrict__ next_w,
    bf16* __restrict__ next_input, long n_pixels, long n_steps, float eps) {
  __shared__ __align__(16) unsigned short tab[2 * kGeluN];
  static_assert(2 * kGeluN * sizeof(unsigned short) % 16 == 0, "table copied in 16-byte pieces");
  for (int i = threadIdx.x; i < static_cast<int>(2 * kGeluN / 8); i += 256)
    reinterpret_cast<uint4*>(tab)[i] = reinterpret_cast<const uint4*>(kGeluBf16Table)[i];

  const int lane = threadIdx.x & 63;
  const int p = lane & 31, g = lane >> 5;
  const int c0 = 8 * g;
  bf16x8 w1[2], w2[4];
  f32x16 b1[2], b2;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int m = 0; m < 8; ++m) w1[blk][m] = static_cast<bf16>(fc1_w[(32 * blk + p) * kPix + c0 + m]);
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int r = 0; r < 16; ++r) b1[blk][r] = fc1_b[32 * blk + 8 * (r >> 2) + 4 * g + (r & 3)];
  // output row p < 16 holds channel ch; rows 16..31 are zero (their weights read row ch % 16)
  const int ch = ((p >> 2) & 1) * 8 + ((p >> 3) & 1) * 4 + (p & 3);
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float w = fc2_w[ch * kHidden + 16 * q + 8 * (m >> 2) + 4 * g + (m & 3)];
      w2[q][m] = static_cast<bf16>(p < kPix ? w : 0.0f);
    }
#pragma unroll
  for (int r = 0; r < 16; ++r) b2[r] = r < 8 ? fc2_b[c0 + r] : 0.0f;
  float nw[8], nnw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    nw[i] = norm_w[c0 + i];
    nnw[i] = next_w[c0 + i];
  }

  const long n_waves = static_cast<long>(gridDim.x) * 4;
  long step = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  PixelShare<TP> nxt;
  if (step < n_steps) load_share(nxt, pixels, branch, mods, min(step * 32 + p, n_pixels - 1), c0);
  __syncthreads();

  for (; step < n_steps; step += n_waves) {
    const PixelShare<TP> cur = nxt;
    if (step + n_waves < n_steps)
      load_share(nxt, pixels, branch, mods, min((step + n_waves) * 32 + p, n_pixels - 1), c0);
    const long idx = step * 32 + p;
    float x[8];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = to_f32(cur.x[i]) + (to_f32(cur.br[i]) * (1.0f + to_f32(cur.s1[i])) + to_f32(cur.t1[i]));
      ss += x[i] * x[i];
    }
    float r = rsqrtf(pair_sum(ss) / kPix + eps);
    bf16x8 hb;
#pragma unroll
    for (int i = 0; i < 8; ++i) hb[i] = static_cast<bf16>((x[i] * r) * nw[i]);
    f32x16 acc[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) acc[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1[blk], hb, b1[blk], 0, 0, 0);
    unsigned worst = 0;
    f32x16 y = b2;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 gb;
      const f32x16& a = acc[q >> 1];
      const int o = 8 * (q & 1);
      gb.x = gelu2_table(a[o + 0], a[o + 1], tab, worst);
      gb.y = gelu2_table(a[o + 2], a[o + 3], tab, worst);
      gb.z = gelu2_table(a[o + 4], a[o + 5], tab, worst);
      gb.w = gelu2_table(a[o + 6], a[o + 7], tab, worst);
      y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2[q], __builtin_bit_cast(bf16x8, gb), y, 0, 0, 0);
    }
    if (__builtin_expect(__any(worst >= kGeluN), 0)) {  // wave-uniform
      y = b2;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        bf16x8 gx;
#pragma unroll
        for (int m = 0; m < 8; ++m) gx[m] = gelu_bf16(acc[q >> 1][8 * (q & 1) + m], tab);
        y = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2[q], gx, y, 0, 0, 0);
      }
    }
    ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = x[i] + (y[i] * (1.0f + to_f32(cur.s2[i])) + to_f32(cur.t2[i]));
      ss += x[i] * x[i];
    }
    r = rsqrtf(pair_sum(ss) / kPix + eps);
    if (idx < n_pixels) {
      store8(pixels + idx * kPix + c0, x);
      float hn[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) hn[i] = (x[i] * r) * nnw[i];
      store8(next_input + idx * kPix + c0, hn);
    }
  }
}

// CO output channels: 3 (the predicted flow) or 1 (the depth head with its 1x1 reducer folded in).
template <int CO>
__global__ __launch_bounds__(256) void unpatchify_head_kernel(const bf16* __restrict__ h, const float* __restrict__ w,
                                                              const float* __restrict__ bias,
                                                              float* __restrict__ out, int batch, int height,
                                                              int width, int patch) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long hw = static_cast<long>(height) * width;
  if (idx >= batch * hw) return;
  const int px_x = static_cast<int>(idx % width);
  const int px_y = static_cast<int>((idx / width) % height);
  const long b = idx / hw;
  const int wp = width / patch;
  const long n_patches = static_cast<long>(height / patch) * wp;
  const long l = static_cast<long>(px_y / patch) * wp + px_x / patch;
  const long q = (b * n_patches + l) * patch * patch + (px_y % patch) * patch + (px_x % patch);
  float v[kPix];
  load8(h + q * kPix, v);
  load8(h + q * kPix + 8, v + 8);
#pragma unroll
  for (int c = 0; c < CO; ++c) {
    float acc = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kPix; ++ch) acc += v[ch] * w[c * kPix + ch];
    out[(b * CO + c) * hw + static_cast<long>(px_y) * width + px_x] = acc + bias[c];
  }
}

inline unsigned blocks_for(long n) { return static_cast<unsigned>((n + 255) / 256); }

template <typename TP>
void launch_patchify(int channels, unsigned blocks, hipStream_t stream, const float* x, int batch, int height,
                     int width, int patch, bf16* patches, long patch_stride, const float* pix_w, const float* pix_b,
                     const float* pos_x, const float* pos_y, const float* norm_w, float eps, TP* pixels,
                     bf16* normed) {
  if (channels == 4)
    patchify_embed_kernel<TP, 4><<<blocks, 256, 0, stream>>>(x, batch, height, width, patch, patches, patch_stride,
                                                             pix_w, pix_b, pos_x, pos_y, norm_w, eps, pixels, normed);
  else
    patchify_embed_kernel<TP, 3><<<blocks, 256, 0, stream>>>(x, batch, height, width, patch, patches, patch_stride,
                                                             pix_w, pix_b, pos_x, pos_y, norm_w, eps, pixels, normed);
}

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_patchify_embed(const float* x, int batch, int channels, int height, int width, int patch,
                                   void* patches,
                                   long patch_stride, const float* pix_w, const float* pix_b, const float* pos_x, const float* pos_y,
                                   const float* norm_weight, float eps, void* pixels, int pixels_dtype,
                                   void* normed, hipStream_t stream) {
  IRIS_REQUIRE(pixels_dtype == IRIS_F32 || pixels_dtype == IRIS_BF16, "patchify_embed: unknown dtype");
  IRIS_REQUIRE(batch >= 0 && patch > 0 && height > 0 && width > 0,
               "patchify_embed: bad sizes");
  IRIS_REQUIRE(height % patch == 0 && width % patch == 0, "input %dx%d is not divisible by patch_size %d", height,
               width, patch);
  IRIS_REQUIRE(channels == 3 || channels == 4, "patchify_embed: 3 or 4 input channels (got %d)", channels);
  IRIS_REQUIRE(patch_stride >= static_cast<long>(channels) * patch * patch,
               "patchify_embed: patch rows shorter than channels*p*p");
  IRIS_REQUIRE(x && patches && pix_w && pix_b && pos_x && pos_y && norm_weight && pixels && normed,
               "patchify_embed: null pointer");
  const long n = static_cast<long>(batch) * height * width;
  if (n == 0) return IRIS_OK;
  if (pixels_dtype == IRIS_F32)
    launch_patchify<float>(channels, blocks_for(n), stream, x, batch, height, width, patch, (bf16*)patches,
                           patch_stride, pix_w, pix_b, pos_x, pos_y, norm_weight, eps, (float*)pixels, (bf16*)normed);
  else
    launch_patchify<bf16>(channels, blocks_for(n), stream, x, batch, height, width, patch, (bf16*)patches,
                          patch_stride, pix_w, pix_b, pos_x, pos_y, norm_weight, eps, (bf16*)pixels, (bf16*)normed);
  return check_launch("patchify_embed");
}

extern "C" int iris_pixel_rms_norm(const void* pixels, int pixels_dtype, void* out, const float* weight,
                                   long n_pixels, float eps, hipStream_t stream) {
  IRIS_REQUIRE(pixels_dtype == IRIS_F32 || pixels_dtype == IRIS_BF16, "pixel_rms_norm: unknown dtype");
  IRIS_REQUIRE(n_pixels >= 0, "pixel_rms_norm: bad size");
  if (n_pixels == 0) return IRIS_OK;  // (empty tensors may come with null data pointers)
  IRIS_REQUIRE(pixels && out && weight, "pixel_rms_norm: null pointer");
  if (pixels_dtype == IRIS_F32)
    pixel_rms_norm_kernel<float><<<blocks_for(n_pixels), 256, 0, stream>>>((const float*)pixels, (bf16*)out, weight,
                                                                           n_pixels, eps);
  else
    pixel_rms_norm_kernel<bf16><<<blocks_for(n_pixels), 256, 0, stream>>>((const bf16*)pixels, (bf16*)out, weight,
                                                                          n_pixels, eps);
  return check_launch("pixel_rms_norm");
}

extern "C" int iris_pixel_mlp(void* pixels, int pixels_dtype, const void* branch, const void* mods,
                              const float* norm_weight, const float* fc1_w, const float* fc1_b, const float* fc2_w,
                              const float* fc2_b, const float* next_norm_weight, void* next_input, long n_pixels,
                              float eps, hipStream_t stream) {
  IRIS_REQUIRE(pixels_dtype == IRIS_F32 || pixels_dtype == IRIS_BF16, "pixel_mlp_: unknown dtype");
  IRIS_REQUIRE(n_pixels >= 0, "pixel_mlp_: bad size");
  if (n_pixels == 0) return IRIS_OK;  // (empty tensors may come with null data pointers)
  IRIS_REQUIRE(pixels && branch && mods && norm_weight && fc1_w && fc1_b && fc2_w && fc2_b && next_norm_weight &&
                   next_input,
               "pixel_mlp_: null pointer");
  // 32 pixels per wave step, 4 waves per workgroup, at most 4 workgroups per CU (each copies
  // the 12 KB GELU table into its LDS once)
  const long n_steps = (n_pixels + 31) / 32;
  const unsigned blocks = static_cast<unsigned>(std::min<long>((n_steps + 3) / 4, 4L * device_cus()));
  if (pixels_dtype == IRIS_F32)
    pixel_mlp_kernel<float><<<blocks, 256, 0, stream>>>(
        (float*)pixels, (const bf16*)branch, (const bf16*)mods, norm_weight, fc1_w, fc1_b, fc2_w, fc2_b,
        next_norm_weight, (bf16*)next_input, n_pixels, n_steps, eps);
  else
    pixel_mlp_kernel<bf16><<<blocks, 256, 0, stream>>>(
        (bf16*)pixels, (const bf16*)branch, (const bf16*)mods, norm_weight, fc1_w, fc1_b, fc2_w, fc2_b,
        next_norm_weight, (bf16*)next_input, n_pixels, n_steps, eps);
  return check_launch("pixel_mlp");
}

extern "C" int iris_unpatchify_head(const void* h, const float* w, const float* bias, float* out, int out_channels,
                                    int batch, int height, int width, int patch, hipStream_t stream) {
  IRIS_REQUIRE(out_channels == 3 || out_channels == 1, "unpatchify_head: 3 or 1 output channels (got %d)",
               out_channels);
  IRIS_REQUIRE(batch >= 0 && patch > 0 && height > 0 && width > 0 && height % patch == 0 && width % patch == 0,
               "unpatchify_head: bad sizes");
  IRIS_REQUIRE(h && w && bias && out, "unpatchify_head: null pointer");
  const long n = static_cast<long>(batch) * height * width;
  if (n == 0) return IRIS_OK;
  if (out_channels == 1)
    unpatchify_head_kernel<1><<<blocks_for(n), 256, 0, stream>>>((const bf16*)h, w, bias, out, batch, height, width,
                                                                 patch);
  else
    unpatchify_head_kernel<3><<<blocks_for(n), 256, 0, stream>>>((const bf16*)h, w, bias, out, batch, height, width,
                                                                 patch);
  return check_launch("unpatchify_head");
}
