// Sampler-side elementwise kernels (FP32) and the timestep features. The update kernels
// evaluate the reference's expressions operation by operation with FMA contraction off,
// so they round exactly like the reference's eager FP32 tensor arithmetic.
#include "iris_common.hpp"

namespace iris {
namespace {

inline unsigned blocks_for(long n) { return static_cast<unsigned>((n + 255) / 256); }

#pragma clang fp contract(off)

__global__ __launch_bounds__(256) void flow_euler_kernel(const float* __restrict__ x, const float* __restrict__ v,
                                                         long n, float sigma, float sigma_next,
                                                         float* __restrict__ x_next, float* __restrict__ clean) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float xi = x[i];
  const float c = xi - sigma * v[i];
  clean[i] = c;
  if (x_next != nullptr) {
    const float one_minus = 1.0f - sigma;
    const float implied_noise = (xi - one_minus * c) / sigma;
    const float one_minus_next = 1.0f - sigma_next;
    x_next[i] = one_minus_next * c + sigma_next * implied_noise;
  }
}

__global__ __launch_bounds__(256) void dpm1_kernel(const float* __restrict__ x, const float* __restrict__ v, long n,
                                                   float s, float c_x, float c_x0, float* __restrict__ x_next) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float xi = x[i];
  const float x0 = xi - s * v[i];
  const float a = c_x * xi;
  const float b = c_x0 * x0;
  x_next[i] = a - b;
}

// Second-order multistep update (first-order when x0_prev is null); also stores this step's
// x0 for the next step's history.
__global__ __launch_bounds__(256) void dpm_kernel(const float* __restrict__ x, const float* __restrict__ v,
                                                  const float* __restrict__ x0_prev, long n, float s, float c_x,
                                                  float c_x0, float c_d, float r0, float* __restrict__ x_next,
                                                  float* __restrict__ x0_out) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float xi = x[i];
  const float x0 = xi - s * v[i];
  if (x0_out) x0_out[i] = x0;
  const float a = c_x * xi;
  const float b = c_x0 * x0;
  float r = a - b;
  if (x0_prev) {
    const float d = (x0 - x0_prev[i]) / r0;
    r = r - c_d * d;
  }
  x_next[i] = r;
}

__global__ __launch_bounds__(256) void cfg_kernel(const float* __restrict__ u, const float* __restrict__ c, long n,
                                                  float scale, float* __restrict__ out) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float ui = u[i];
  const float d = c[i] - ui;
  out[i] = ui + scale * d;
}

__global__ __launch_bounds__(256) void clamp_kernel(const float* __restrict__ x, long n, float lo, float hi,
                                                    float* __restrict__ out) {
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  out[i] = v != v ? v : fminf(fmaxf(v, lo), hi);
}

__global__ __launch_bounds__(256) void timestep_features_kernel(const float* __restrict__ t,
                                                                const float* __restrict__ freqs, int batch,
                                                                int half, float* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= batch * half) return;
  const int b = i / half;
  const int j = i - b * half;
  const float phase = t[b] * freqs[j];
  out[b * 2 * half + j] = cosf(phase);
  out[b * 2 * half + half + j] = sinf(phase);
}

#pragma clang fp contract(on)

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_flow_euler(const float* x, const float* v, long n, float sigma, float sigma_next,
                               float* x_next, float* clean, hipStream_t stream) {
  IRIS_REQUIRE(n >= 0 && x && v && clean, "flow_euler: bad arguments");
  IRIS_REQUIRE(sigma > 0.0f, "flow_euler: sigma must be positive");
  if (n == 0) return IRIS_OK;
  flow_euler_kernel<<<blocks_for(n), 256, 0, stream>>>(x, v, n, sigma, sigma_next, x_next, clean);
  return check_launch("flow_euler");
}

extern "C" int iris_dpm1_update(const float* x, const float* v, long n, float s, float c_x, float c_x0,
                                float* x_next, hipStream_t stream) {
  IRIS_REQUIRE(n >= 0 && x && v && x_next, "dpm1_update: bad arguments");
  if (n == 0) return IRIS_OK;
  dpm1_kernel<<<blocks_for(n), 256, 0, stream>>>(x, v, n, s, c_x, c_x0, x_next);
  return check_launch("dpm1_update");
}

extern "C" int iris_dpm_update(const float* x, const float* v, const float* x0_prev, long n, float s, float c_x,
                               float c_x0, float c_d, float r0, float* x_next, float* x0_out, hipStream_t stream) {
  IRIS_REQUIRE(n >= 0 && x && v && x_next, "dpm_update: bad arguments");
  IRIS_REQUIRE(!x0_prev || r0 != 0.0f, "dpm_update: the step ratio r0 must be nonzero");
  IRIS_REQUIRE(x_next != x && x_next != v && (!x0_out || (x0_out != x && x0_out != v && x0_out != x_next)) &&
                   (!x0_prev || (x0_prev != x_next && x0_prev != x0_out)),
               "dpm_update: outputs must not alias the inputs or each other");
  if (n == 0) return IRIS_OK;
  dpm_kernel<<<blocks_for(n), 256, 0, stream>>>(x, v, x0_prev, n, s, c_x, c_x0, c_d, r0, x_next, x0_out);
  return check_launch("dpm_update");
}

extern "C" int iris_cfg_combine(const float* v_uncond, const float* v_cond, long n, float scale, float* out,
                                hipStream_t stream) {
  IRIS_REQUIRE(n >= 0 && v_uncond && v_cond && out, "cfg_combine: bad arguments");
  if (n == 0) return IRIS_OK;
  cfg_kernel<<<blocks_for(n), 256, 0, stream>>>(v_uncond, v_cond, n, scale, out);
  return check_launch("cfg_combine");
}

extern "C" int iris_clamp(const float* x, long n, float lo, float hi, float* out, hipStream_t stream) {
  IRIS_REQUIRE(n >= 0 && x && out && lo <= hi, "clamp: bad arguments");
  if (n == 0) return IRIS_OK;
  clamp_kernel<<<blocks_for(n), 256, 0, stream>>>(x, n, lo, hi, out);
  return check_launch("clamp");
}

extern "C" int iris_timestep_features(const float* t, const float* freqs, int batch, int half, float* out,
                                      hipStream_t stream) {
  IRIS_REQUIRE(batch >= 0 && half > 0 && t && freqs && out, "timestep_features: bad arguments");
  if (batch == 0) return IRIS_OK;
  timestep_features_kernel<<<blocks_for(static_cast<long>(batch) * half), 256, 0, stream>>>(t, freqs, batch, half,
                                                                                          out);
  return check_launch("timestep_features");
}
