// Pixel-stage bandwidth kernels: patchify + pixel embedding, the per-pixel RMSNorm, the
// post-modulated PiT tail (norm, 16 -> 64 -> 16 exact-GELU MLP, both modulated residual
// adds, next block's norm) and the 16 -> 3 head with unpatchify. One thread per pixel,
// all math in FP32; BF16 only where the value is stored.
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

// Exact GELU a Phi(a), Phi(a) = erfc(-a / sqrt 2) / 2, with erfc(z), z >= 0, by the Chebyshev fit of
// Press et al., Numerical Recipes in C (2nd ed.) sec. 6.2 ("erfcc", fractional error < 1.2e-7
// everywhere): erfc(z) = t exp(-z^2 + P(t)), t = 1 / (1 + z / 2), P a degree-9 polynomial; and
// Phi(a) = 1 - erfc(|a| / sqrt 2) / 2 for a >= 0. The tail a << 0 keeps full relative precision:
// z^2 = a^2 / 2 is carried as hi + lo (exact square split by an fma, halved exactly), and
// exp(-hi) is taken as exp2 of hi log2(e) with the product's rounding error moved into the
// small second factor. About twenty VALU instructions instead of the library erfcf's fifty.
__device__ __forceinline__ float gelu_erf(float a) {
  constexpr float kLog2e = 1.44269504088896341f;
  const float z = fabsf(a) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float poly = 0.17087277f;
  poly = fmaf(t, poly, -0.82215223f);
  poly = fmaf(t, poly, 1.48851587f);
  poly = fmaf(t, poly, -1.13520398f);
  poly = fmaf(t, poly, 0.27886807f);
  poly = fmaf(t, poly, -0.18628806f);
  poly = fmaf(t, poly, 0.09678418f);
  poly = fmaf(t, poly, 0.37409196f);
  poly = fmaf(t, poly, 1.00002368f);
  const float aa = a * a;
  const float hi = 0.5f * aa;                      // z^2 = hi + lo
  const float lo = 0.5f * fmaf(a, a, -aa);
  const float small = fmaf(t, poly, -1.26551223f) - lo;
  const float p = hi * kLog2e;
  const float p_err = fmaf(hi, kLog2e, -p);        // hi log2(e) = p + p_err
  const float q = (0.5f * t) * __builtin_amdgcn_exp2f(-p) * __builtin_amdgcn_exp2f(fmaf(small, kLog2e, -p_err));
  return a * (a >= 0.0f ? 1.0f - q : q);
}

template <typename TP>
__global__ __launch_bounds__(256) void pixel_mlp_kernel(
    TP* __restrict__ pixels, const bf16* __restrict__ branch, const bf16* __restrict__ mods,
    const float* __restrict__ norm_w, const float* __restrict__ fc1_w, const float* __restrict__ fc1_b,
    const float* __restrict__ fc2_w, const float* __restrict__ fc2_b, const float* __restrict__ next_w,
    bf16* __restrict__ next_input, long n_pixels, float eps) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n_pixels) return;
  float m[4 * kPix];
#pragma unroll
  for (int i = 0; i < 8; ++i) load8(mods + idx * 4 * kPix + 8 * i, m + 8 * i);
  float br[kPix], x[kPix];
  load8(branch + idx * kPix, br);
  load8(branch + idx * kPix + 8, br + 8);
  load8(pixels + idx * kPix, x);
  load8(pixels + idx * kPix + 8, x + 8);
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kPix; ++c) {
    x[c] = x[c] + (br[c] * (1.0f + m[c]) + m[kPix + c]);  // scale1, shift1
    ss += x[c] * x[c];
  }
  float r = rsqrtf(ss / kPix + eps);
  float h[kPix], out[kPix];
#pragma unroll
  for (int c = 0; c < kPix; ++c) {
    h[c] = (x[c] * r) * norm_w[c];
    out[c] = fc2_b[c];
  }
  for (int j = 0; j < kHidden; ++j) {
    float a = fc1_b[j];
#pragma unroll
    for (int c = 0; c < kPix; ++c) a += fc1_w[j * kPix + c] * h[c];
    const float g = gelu_erf(a);
#pragma unroll
    for (int c = 0; c < kPix; ++c) out[c] += fc2_w[c * kHidden + j] * g;
  }
  ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kPix; ++c) {
    x[c] = x[c] + (out[c] * (1.0f + m[2 * kPix + c]) + m[3 * kPix + c]);  // scale2, shift2
    ss += x[c] * x[c];
  }
  store8(pixels + idx * kPix, x);
  store8(pixels + idx * kPix + 8, x + 8);
  r = rsqrtf(ss / kPix + eps);
#pragma unroll
  for (int c = 0; c < kPix; ++c) h[c] = (x[c] * r) * next_w[c];
  store8(next_input + idx * kPix, h);
  store8(next_input + idx * kPix + 8, h + 8);
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
  IRIS_REQUIRE(pixels && out && weight, "pixel_rms_norm: null pointer");
  if (n_pixels == 0) return IRIS_OK;
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
  IRIS_REQUIRE(pixels && branch && mods && norm_weight && fc1_w && fc1_b && fc2_w && fc2_b && next_norm_weight &&
                   next_input,
               "pixel_mlp_: null pointer");
  if (n_pixels == 0) return IRIS_OK;
  if (pixels_dtype == IRIS_F32)
    pixel_mlp_kernel<float><<<blocks_for(n_pixels), 256, 0, stream>>>(
        (float*)pixels, (const bf16*)branch, (const bf16*)mods, norm_weight, fc1_w, fc1_b, fc2_w, fc2_b,
        next_norm_weight, (bf16*)next_input, n_pixels, eps);
  else
    pixel_mlp_kernel<bf16><<<blocks_for(n_pixels), 256, 0, stream>>>(
        (bf16*)pixels, (const bf16*)branch, (const bf16*)mods, norm_weight, fc1_w, fc1_b, fc2_w, fc2_b,
        next_norm_weight, (bf16*)next_input, n_pixels, eps);
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
