// Shared types, vector helpers and error reporting for the Iris MI355X (gfx950) kernels.
//
// Every kernel in this library works on caller-owned device memory; entry points
// validate their arguments on the host, launch asynchronously on the given
// stream and return IRIS_OK or a negative IRIS_E_* code (message retrievable
// with iris_last_error()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/iris_hip.h"

namespace iris {

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---- host-side error state --------------------------------------------------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

#define IRIS_REQUIRE(cond, ...)                      \
  do {                                               \
    if (!(cond)) return ::iris::fail(IRIS_E_INVALID, __VA_ARGS__); \
  } while (0)

inline bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Compute units of the current device (launch shapes that place one workgroup per CU).
inline int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    cached[dev] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0
                      ? cus
                      : 256;
  }
  return cached[dev];
}

// ---- device helpers ----------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// 4-element loads / stores returning / taking FP32.
__device__ __forceinline__ f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{to_f32(v[0]), to_f32(v[1]), to_f32(v[2]), to_f32(v[3])};
}
__device__ __forceinline__ void store4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void store4(bf16* p, f32x4 v) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{from_f32<bf16>(v[0]), from_f32<bf16>(v[1]), from_f32<bf16>(v[2]),
                                         from_f32<bf16>(v[3])};
}

// 8-element loads / stores.
__device__ __forceinline__ void load8(const float* p, float* out) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = a[i];
    out[4 + i] = b[i];
  }
}
__device__ __forceinline__ void load8(const bf16* p, float* out) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = to_f32(v[i]);
}
__device__ __forceinline__ void store8(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}
__device__ __forceinline__ void store8(bf16* p, const float* v) {
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = from_f32<bf16>(v[i]);
  *reinterpret_cast<bf16x8*>(p) = o;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Position of token slot i inside its group of 16 in the V^T layout the attention kernel reads:
// the middle two 4-token quads are swapped (0-3, 8-11, 4-7, 12-15), so that the 8 keys one
// MFMA lane needs (4 g .. 4 g + 3 and 8 + 4 g .. 8 + 4 g + 3) are contiguous. An involution.
__device__ __forceinline__ int vt_slot(int i) {
  const int quad = (i >> 2) & 3;
  return (i & ~15) | ((quad == 1 ? 2 : quad == 2 ? 1 : quad) << 2) | (i & 3);
}

// Per-head RMSNorm + rotary embedding of one 128-wide head: y = rope((a / rms) * w), rms over
// the 128 values (+ eps inside the root), pair j = (2 j, 2 j + 1) rotated by (c[j], s[j]) of its
// position. The head is held as 16 chunks of 8 values (chunk s: elements 8 s .. 8 s + 7, rotary
// pairs 4 s .. 4 s + 3); the squares are summed per chunk in element order, and the 16 chunk sums
// combined as an xor butterfly over chunks 8, 4, 2, 1 apart (head_norm_rope: one chunk per lane
// of an aligned 16-lane group, every lane of which must take part; head_sum_tree: the same
// additions in one thread, equal bits).
// (The fused multiply-adds are spelled out: left to contraction, the compiler fused a different
// product of a two-product sum in different callers, one BF16 step apart now and then.)
__device__ __forceinline__ float head_chunk_sq(const float (&a)[8]) {
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(a[e], a[e], ss);
  return ss;
}
__device__ __forceinline__ float head_sum_tree(const float (&ss)[16]) {
  float v1[8], v2[4], v3[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) v1[i] = ss[i] + ss[i + 8];
#pragma unroll
  for (int i = 0; i < 4; ++i) v2[i] = v1[i] + v1[i + 4];
#pragma unroll
  for (int i = 0; i < 2; ++i) v3[i] = v2[i] + v2[i + 2];
  return v3[0] + v3[1];
}
__device__ __forceinline__ float head_rms_scale(float sum_sq, float eps) { return rsqrtf(sum_sq / 128.0f + eps); }
__device__ __forceinline__ void head_scale_rope(const float (&a)[8], float r, const float (&w)[8], const f32x4& c,
                                                const f32x4& s, float (&y)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float a0 = (a[2 * p] * r) * w[2 * p];
    const float a1 = (a[2 * p + 1] * r) * w[2 * p + 1];
    y[2 * p] = __builtin_fmaf(a0, c[p], -(a1 * s[p]));
    y[2 * p + 1] = __builtin_fmaf(a0, s[p], a1 * c[p]);
  }
}
__device__ __forceinline__ void head_norm_rope(const float (&a)[8], const float (&w)[8], const f32x4& c,
                                               const f32x4& s, float eps, float (&y)[8]) {
  head_scale_rope(a, head_rms_scale(group_sum<16>(head_chunk_sq(a)), eps), w, c, s, y);
}

// x sigmoid(x) and sigmoid(x) with the hardware reciprocal (~1 ulp) in place of an IEEE division,
// which costs about ten instructions per element in the GEMM and attention epilogues.
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Map the hardware id to a logical id so that consecutive logical ids run on
// the same XCD; neighbouring logical tiles then share operands in one L2.
__device__ __forceinline__ int xcd_remap(int wg, int total) {
  const int xcd = wg & 7;
  const int local = wg >> 3;
  const int base = total >> 3;
  const int rem = total & 7;
  return xcd * base + (xcd < rem ? xcd : rem) + local;
}

// Raw buffer resources: word 3 of a gfx9-family buffer descriptor (32-bit dwords, no swizzle).
// A buffer load takes one 32-bit VGPR byte offset and an SGPR offset, and reads past the
// resource's size return zeros instead of faulting.
constexpr int kBufferFlags = 0x00020000;

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane (lds wave-uniform). (A
// non-template device function: the host compilation pass never instantiates it, which it would
// reject for the LDS address-space cast, and the kernels calling it keep their launch stubs.)
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, bf16* lds, int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0,
                                           0);
}

}  // namespace iris
