// BF16-weight matrix-vector products for the per-step conditioning: the timestep MLP and
// the shared adaLN cores (M = batch <= 4 per launch). HBM-bound on the weight read: each
// wave streams whole weight rows with 16-byte loads while the (activated) input vectors sit
// in LDS, staged once per workgroup.
#include "iris_common.hpp"

namespace iris {
namespace {

constexpr int kMaxBatch = 4;
constexpr int kRowsPerWave = 2;
constexpr int kRowsPerBlock = 4 * kRowsPerWave;

__global__ __launch_bounds__(256) void gemv_kernel(const bf16* __restrict__ w, const float* __restrict__ x,
                                                   int nb, int n, int k, const float* __restrict__ bias,
                                                   const float* __restrict__ extra, int n_extra,
                                                   float* __restrict__ out, long out_bstride, long out_jstride,
                                                   int in_act, int out_act) {
  extern __shared__ float xs[];  // nb * k
  for (int i = threadIdx.x; i < nb * k; i += 256) {
    const float v = x[i];
    xs[i] = in_act == IRIS_ACT_SILU ? silu(v) : v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int row0 = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6) * kRowsPerWave;
  const int chunks = k >> 3;
#pragma unroll
  for (int rr = 0; rr < kRowsPerWave; ++rr) {
    const int row = row0 + rr;
    if (row >= n) break;  // uniform across the wave
    float acc[kMaxBatch] = {0.0f, 0.0f, 0.0f, 0.0f};
    const bf16* wr = w + static_cast<long>(row) * k;
    for (int c = lane; c < chunks; c += kWave) {
      float wv[8];
      load8(wr + 8 * c, wv);
#pragma unroll
      for (int b = 0; b < kMaxBatch; ++b) {
        if (b < nb) {
          const float* xb = xs + b * k + 8 * c;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[b] += wv[e] * xb[e];
        }
      }
    }
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) {
      if (b >= nb) break;
      float y = wave_sum(acc[b]);  // (every lane holds the sum)
      if (bias) y += bias[row];
      if (out_act == IRIS_ACT_SILU) y = silu(y);
      if (n_extra == 0) {
        if (lane == 0) out[b * out_bstride + row] = y;
      } else {  // the per-block copies, one per lane
        for (int j = lane; j < n_extra; j += kWave)
          out[j * out_jstride + b * out_bstride + row] = y + extra[static_cast<long>(j) * n + row];
      }
    }
  }
}

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_gemv_bf16(const void* w, const float* x, int batch, int n, int k, const float* bias,
                              const float* extra_bias, int n_extra, float* out, int in_act, int out_act,
                              hipStream_t stream) {
  IRIS_REQUIRE(batch >= 0 && n > 0 && k > 0 && k % 8 == 0 && k <= 4096, "gemv: need k %% 8 == 0 and k <= 4096");
  IRIS_REQUIRE(n_extra >= 0 && (n_extra == 0 || extra_bias), "gemv: extra biases missing");
  IRIS_REQUIRE((in_act == IRIS_ACT_NONE || in_act == IRIS_ACT_SILU) &&
                   (out_act == IRIS_ACT_NONE || out_act == IRIS_ACT_SILU),
               "gemv: unknown activation");
  IRIS_REQUIRE(w && x && out, "gemv: null pointer");
  IRIS_REQUIRE(aligned(w, 16), "gemv: weight must be 16-byte aligned");
  const long out_bstride = n;
  const long out_jstride = static_cast<long>(batch) * n;
  for (int b0 = 0; b0 < batch; b0 += kMaxBatch) {
    const int nb = batch - b0 < kMaxBatch ? batch - b0 : kMaxBatch;
    const dim3 grid((n + kRowsPerBlock - 1) / kRowsPerBlock);
    const size_t lds = static_cast<size_t>(nb) * k * sizeof(float);
    gemv_kernel<<<grid, 256, lds, stream>>>((const bf16*)w, x + static_cast<long>(b0) * k, nb, n, k, bias,
                                            extra_bias, n_extra, out + static_cast<long>(b0) * n, out_bstride,
                                            out_jstride, in_act, out_act);
    const int rc = check_launch("gemv");
    if (rc) return rc;
  }
  return IRIS_OK;
}
