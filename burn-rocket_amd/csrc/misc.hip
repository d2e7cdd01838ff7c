// Format conversions and activation quantizers on the GPU.
//
// These are the host-side steps around every call in the reference
// (f32_to_f16_par / f16_to_f32_par ext.rs:2144-2170, quantize_i8_rows
// ext.rs:1017-1029 with quantize_row_groups host.rs:77-90, the QAT static
// quantizer and epilogue ext.rs:1236-1373), moved next to the data.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

__global__ void f32_to_f16_kernel(const float *__restrict__ x, f16 *__restrict__ y, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    floatx4 v = *(const floatx4 *)(x + i);
    half4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *(half4 *)(y + i) = h;
  } else {
    for (; i < n; ++i) y[i] = (f16)x[i];
  }
}

__global__ void f16_to_f32_kernel(const f16 *__restrict__ x, float *__restrict__ y, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    half4 h = *(const half4 *)(x + i);
    *(floatx4 *)(y + i) = floatx4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  } else {
    for (; i < n; ++i) y[i] = (float)x[i];
  }
}

// f32 -> fp16 that also sets *flag to 1 when a converted value is not finite
// (an input outside fp16's range, or not finite itself).
__global__ void f32_to_f16_checked_kernel(const float *__restrict__ x, f16 *__restrict__ y, int64_t n,
                                          int *__restrict__ flag) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  bool bad = false;
  if (i + 3 < n) {
    floatx4 v = *(const floatx4 *)(x + i);
    half4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *(half4 *)(y + i) = h;
#pragma unroll
    for (int e = 0; e < 4; ++e) bad |= !isfinite((float)h[e]);
  } else {
    for (; i < n; ++i) {
      const f16 h = (f16)x[i];
      y[i] = h;
      bad |= !isfinite((float)h);
    }
  }
  if (bad) *flag = 1;
}

hipError_t rk_launch_f32_to_f16_checked(const float *x, void *y, int64_t n, int *flag, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(f32_to_f16_checked_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, x, (f16 *)y, n, flag);
  return hipGetLastError();
}

hipError_t rk_launch_f32_to_f16(const float *x, void *y, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  // Vector path needs 16-byte aligned rows of 4; callers pass whole buffers.
  int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, x, (f16 *)y, n);
  return hipGetLastError();
}

// Element type conversion between f32, fp16 and bf16 (RK_DTYPE_*), rounding
// to nearest even, four elements per thread.
template <int SRC, int DST>
__global__ __launch_bounds__(256) void cast_kernel(const void *__restrict__ x, void *__restrict__ y,
                                                   int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i0 + e < n) dt_store<DST>(y, i0 + e, dt_load<SRC>(x, i0 + e));
}

template <int SRC>
static hipError_t launch_cast_from(const void *x, void *y, int64_t n, int dst, hipStream_t st) {
  const dim3 grid((unsigned)((n + 1023) / 1024)), block(256);
  switch (dst) {
    case RK_DTYPE_F32: hipLaunchKernelGGL((cast_kernel<SRC, RK_DTYPE_F32>), grid, block, 0, st, x, y, n); break;
    case RK_DTYPE_F16: hipLaunchKernelGGL((cast_kernel<SRC, RK_DTYPE_F16>), grid, block, 0, st, x, y, n); break;
    case RK_DTYPE_BF16: hipLaunchKernelGGL((cast_kernel<SRC, RK_DTYPE_BF16>), grid, block, 0, st, x, y, n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t rk_launch_cast(const void *x, int src, void *y, int dst, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  switch (src) {
    case RK_DTYPE_F32: return launch_cast_from<RK_DTYPE_F32>(x, y, n, dst, st);
    case RK_DTYPE_F16: return launch_cast_from<RK_DTYPE_F16>(x, y, n, dst, st);
    case RK_DTYPE_BF16: return launch_cast_from<RK_DTYPE_BF16>(x, y, n, dst, st);
  }
  return hipErrorInvalidValue;
}

__global__ void f32_to_f16_rows_kernel(const float *__restrict__ x, int64_t n, int64_t k,
                                       int grp_stride, int grp_off, f16 *__restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * k) return;
  const int64_t r = i / k, c = i % k;
  y[((r / 16) * grp_stride + grp_off + r % 16) * k + c] = (f16)x[i];
}

hipError_t rk_launch_f32_to_f16_rows(const float *x, int64_t n, int64_t k, int grp_stride,
                                     int grp_off, void *out, hipStream_t st) {
  if (n * k <= 0) return hipSuccess;
  hipLaunchKernelGGL(f32_to_f16_rows_kernel, dim3((unsigned)((n * k + 255) / 256)), dim3(256), 0, st,
                     x, n, k, grp_stride, grp_off, (f16 *)out);
  return hipGetLastError();
}

hipError_t rk_launch_f16_to_f32(const void *x, float *y, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, (const f16 *)x, y, n);
  return hipGetLastError();
}

// One workgroup per row. Group maxima are reduced with LDS atomics on the
// f32 bit pattern (all values are >= 0, so integer order is float order).
constexpr int QROW_THREADS = 256;
constexpr int QROW_MAX_GROUPS = 1024;

__global__ __launch_bounds__(QROW_THREADS) void quantize_rows_kernel(
    const float *__restrict__ x, int64_t k, int64_t group, int8_t *__restrict__ q,
    float *__restrict__ scale) {
  __shared__ unsigned int amax[QROW_MAX_GROUPS];
  __shared__ float inv[QROW_MAX_GROUPS];
  const int64_t row = blockIdx.x;
  const int ng = (int)(k / group);
  const float *xr = x + row * k;
  for (int g = threadIdx.x; g < ng; g += QROW_THREADS) amax[g] = 0u;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < k; i += QROW_THREADS) {
    float a = fabsf(xr[i]);
    atomicMax(&amax[i / group], __float_as_uint(a));
  }
  __syncthreads();
  for (int g = threadIdx.x; g < ng; g += QROW_THREADS) {
    float s = fmaxf(__uint_as_float(amax[g]) / 127.0f, 1e-12f);
    scale[row * ng + g] = s;
    inv[g] = 1.0f / s;
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < k; i += QROW_THREADS) {
    float v = roundf(xr[i] * inv[i / group]);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[row * k + i] = (int8_t)(int)v;
  }
}

// Per-token form (one scale per row, k % 4 == 0): one wave per row, four
// rows per workgroup. The row is read once into registers as float4s, the
// maximum is reduced across the wave (max is exact in any order), and the
// codes are written four to a 32-bit store. Same arithmetic as above.
constexpr int QTOK_MAX_VEC = 16;  // float4 per lane: rows up to 4096 values
__global__ __launch_bounds__(256) void quantize_tokens_kernel(const float *__restrict__ x,
                                                              int64_t m, int64_t k,
                                                              int8_t *__restrict__ q,
                                                              float *__restrict__ scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int nv = (int)(k / 4);
  const floatx4 *xr = (const floatx4 *)(x + row * k);
  floatx4 v[QTOK_MAX_VEC];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < QTOK_MAX_VEC; ++i) {
    const int j = lane + 64 * i;
    v[i] = j < nv ? xr[j] : floatx4{0.f, 0.f, 0.f, 0.f};
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3]))));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float s = fmaxf(amax / 127.0f, 1e-12f);
  const float inv = 1.0f / s;
  if (lane == 0) scale[row] = s;
  uint32_t *qr = (uint32_t *)(q + row * k);
#pragma unroll
  for (int i = 0; i < QTOK_MAX_VEC; ++i) {
    const int j = lane + 64 * i;
    if (j < nv) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float c = roundf(v[i][e] * inv);
        c = fminf(fmaxf(c, -127.0f), 127.0f);
        packed |= (uint32_t)(uint8_t)(int8_t)(int)c << (8 * e);
      }
      qr[j] = packed;
    }
  }
}

// 32-value groups (K % 32 == 0): each lane quantizes 8 consecutive values, so
// four neighbouring lanes hold one group (groups never straddle a row) and
// the group maximum is two lane swaps. Same arithmetic as above.
__global__ __launch_bounds__(256) void quantize_g32_kernel(const float *__restrict__ x, int64_t n8,
                                                           int8_t *__restrict__ q,
                                                           float *__restrict__ scale) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n8) return;  // n8 % 4 == 0: a group's four lanes leave together
  const floatx4 a = ((const floatx4 *)x)[2 * t], b = ((const floatx4 *)x)[2 * t + 1];
  float amax = fmaxf(fmaxf(fmaxf(fabsf(a[0]), fabsf(a[1])), fmaxf(fabsf(a[2]), fabsf(a[3]))),
                     fmaxf(fmaxf(fabsf(b[0]), fabsf(b[1])), fmaxf(fabsf(b[2]), fabsf(b[3]))));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 4));
  const float s = fmaxf(amax / 127.0f, 1e-12f);
  const float inv = 1.0f / s;
  if ((t & 3) == 0) scale[t >> 2] = s;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float c = roundf((e < 4 ? a[e] : b[e - 4]) * inv);
    c = fminf(fmaxf(c, -127.0f), 127.0f);
    w[e >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)c << (8 * (e & 3));
  }
  ((uintx2 *)q)[t] = uintx2{w[0], w[1]};
}

hipError_t rk_launch_quantize_rows(const float *x, int64_t m, int64_t k, int64_t group,
                                   int8_t *q, float *scale, hipStream_t st) {
  if (m <= 0) return hipSuccess;
  if (group == 32 && k % 32 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 8) == 0 &&
      ((uintptr_t)scale % 4) == 0) {
    const int64_t n8 = m * k / 8;
    hipLaunchKernelGGL(quantize_g32_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, x,
                       n8, q, scale);
    return hipGetLastError();
  }
  if (group == k && k % 4 == 0 && k <= 4 * 64 * QTOK_MAX_VEC &&
      ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 4) == 0) {
    hipLaunchKernelGGL(quantize_tokens_kernel, dim3((unsigned)((m + 3) / 4)), dim3(256), 0, st, x,
                       m, k, q, scale);
    return hipGetLastError();
  }
  if (k / group > QROW_MAX_GROUPS) return hipErrorInvalidValue;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)m), dim3(QROW_THREADS), 0, st, x, k,
                     group, q, scale);
  return hipGetLastError();
}

// QAT activation grid: ties-to-even, clamped to [-128, 127]. in_scale == 0
// selects the per-row dynamic scale max(amax/127, 1e-12).
__global__ __launch_bounds__(QROW_THREADS) void quantize_static_kernel(
    const float *__restrict__ x, int64_t k, float in_scale, int8_t *__restrict__ q,
    float *__restrict__ row_scale) {
  __shared__ unsigned int amax;
  __shared__ float inv_s;
  const int64_t row = blockIdx.x;
  const float *xr = x + row * k;
  if (threadIdx.x == 0) amax = 0u;
  __syncthreads();
  if (in_scale == 0.0f) {
    for (int64_t i = threadIdx.x; i < k; i += QROW_THREADS)
      atomicMax(&amax, __float_as_uint(fabsf(xr[i])));
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float rs = in_scale;
    if (in_scale == 0.0f) rs = fmaxf(__uint_as_float(amax) / 127.0f, 1e-12f);
    row_scale[row] = rs;
    inv_s = 1.0f / rs;
  }
  __syncthreads();
  const float inv = inv_s;
  for (int64_t i = threadIdx.x; i < k; i += QROW_THREADS) {
    float v = rintf(xr[i] * inv);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    q[row * k + i] = (int8_t)(int)v;
  }
}

hipError_t rk_launch_quantize_static(const float *x, int64_t m, int64_t k, float in_scale,
                                     int8_t *q, float *row_scale, hipStream_t st) {
  if (m <= 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_static_kernel, dim3((unsigned)m), dim3(QROW_THREADS), 0, st, x, k,
                     in_scale, q, row_scale);
  return hipGetLastError();
}

__global__ void qat_epilogue_kernel(const int32_t *__restrict__ acc,
                                    const float *__restrict__ row_scale,
                                    const float *__restrict__ w_scale, int64_t m, int64_t n,
                                    float out_scale, float *__restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m * n) return;
  const int64_t r = i / n, c = i % n;
  float v = (float)acc[i] * (row_scale[r] * w_scale[c]);
  if (out_scale != 0.0f) {
    const float out_inv = 1.0f / out_scale;
    float code = fminf(fmaxf(rintf(v * out_inv), -128.0f), 127.0f);
    v = code * out_scale;
  }
  y[i] = v;
}

hipError_t rk_launch_qat_epilogue(const int32_t *acc, const float *row_scale,
                                  const float *w_scale, int64_t m, int64_t n, float out_scale,
                                  float *y, hipStream_t st) {
  if (m * n <= 0) return hipSuccess;
  hipLaunchKernelGGL(qat_epilogue_kernel, dim3((unsigned)((m * n + 255) / 256)), dim3(256), 0,
                     st, acc, row_scale, w_scale, m, n, out_scale, y);
  return hipGetLastError();
}

// GGUF Q8_0 quantizer (llama.cpp rule, crates/rocket-npu/src/bin/q8_bench.rs:
// 200-220): per 32-value block d = f16(amax/127); codes are quantized against
// the stored f32(d) with inv = d > 0 ? 1/d : 0, round-half-away, clamp ±127.
// One thread per block. Source row r of block column b goes to destination
// row (r / 32)·grp_stride + grp_off + r % 32, which lets the gate and up
// projections of an expert interleave per 32-row slice.
__global__ void q8_0_quantize_kernel(const float *__restrict__ w, int64_t n, int64_t k,
                                     int grp_stride, int grp_off, int8_t *__restrict__ codes,
                                     float *__restrict__ scales, int ws_stride, int frag) {
  const int64_t nb = k / 32;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * nb) return;
  const int64_t r = i / nb, b = i % nb;
  const float *src = w + r * k + b * 32;
  float amax = 0.f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(src[j]));
  const float scale = (float)(f16)(amax / 127.0f);
  const float inv = scale > 0.f ? 1.0f / scale : 0.f;
  const int64_t dr = (r / 16) * grp_stride + grp_off + (r % 16);
  for (int j = 0; j < 32; ++j) {
    float v = roundf(src[j] * inv);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    codes[q8_code_offset(dr, b, j, k, ws_stride, frag)] = (int8_t)(int)v;
  }
  scales[q8_scale_offset(dr, b, ws_stride, frag)] = scale;
}

hipError_t rk_launch_q8_0_quantize(const float *w, int64_t n, int64_t k, int grp_stride,
                                   int grp_off, int8_t *codes, float *scales, int ws_stride,
                                   bool frag, hipStream_t st) {
  const int64_t total = n * (k / 32);
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(q8_0_quantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     w, n, k, grp_stride, grp_off, codes, scales, ws_stride, (int)frag);
  return hipGetLastError();
}

// GGUF Q8_0 blocks (34 bytes: f16 d little-endian, then 32 int8 codes;
// src/util/gguf.rs:125-200) already on the device → codes and f32 scales in
// the layout rk_launch_q8_0_quantize writes (rows remapped the same way). One
// thread per block; blocks are 2-byte aligned, so they are read as 16-bit words.
__device__ __forceinline__ float f16_bits_to_f32_exact(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1fu) return __uint_as_float(sign | 0x7f800000u | (m << 13));
  if (e != 0) return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
  // zero or subnormal: m·2^-24, exact in f32
  return __uint_as_float(sign) + (sign ? -1.0f : 1.0f) * (float)m * 5.9604644775390625e-08f;
}

__global__ void q8_0_unpack_kernel(const uint16_t *__restrict__ blocks, int64_t n, int64_t k,
                                   int grp_stride, int grp_off, int8_t *__restrict__ codes,
                                   float *__restrict__ scales, int ws_stride, int frag) {
  const int64_t nb = k / 32;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * nb) return;
  const int64_t r = i / nb, b = i % nb;
  const uint16_t *blk = blocks + i * 17;  // 34 bytes = 17 16-bit words
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = (uint32_t)blk[1 + 2 * j] | ((uint32_t)blk[2 + 2 * j] << 16);
  const int64_t dr = (r / 16) * grp_stride + grp_off + (r % 16);
  // codes 0..15 and 16..31 are each 16 contiguous bytes in both layouts
  *(uintx4 *)(codes + q8_code_offset(dr, b, 0, k, ws_stride, frag)) = uintx4{w[0], w[1], w[2], w[3]};
  *(uintx4 *)(codes + q8_code_offset(dr, b, 16, k, ws_stride, frag)) = uintx4{w[4], w[5], w[6], w[7]};
  scales[q8_scale_offset(dr, b, ws_stride, frag)] = f16_bits_to_f32_exact(blk[0]);
}

hipError_t rk_launch_q8_0_unpack(const void *blocks, int64_t n, int64_t k, int grp_stride,
                                 int grp_off, int8_t *codes, float *scales, int ws_stride,
                                 bool frag, hipStream_t st) {
  const int64_t total = n * (k / 32);
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(q8_0_unpack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     (const uint16_t *)blocks, n, k, grp_stride, grp_off, codes, scales, ws_stride,
                     (int)frag);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// MLP glue: out = silu(gate)·up or gelu_tanh(gate)·up elementwise
// (rocket_silu_mul / rocket_gelu_mul, ext.rs:603-608 and 1057-1090, with the
// formulas of host.rs:12-39), computed in f32 in the reference's order with
// no FMA contraction, inputs and output in f32, fp16 or bf16 (the output in
// the input type, rounded to nearest even). Each thread handles 16 bytes of
// each input when all three pointers are 16-byte aligned, else one element.
// ---------------------------------------------------------------------------
namespace {
__device__ __forceinline__ float glue_silu_mul(float g, float u) {
#pragma clang fp contract(off)
  const float sigmoid = 1.0f / (1.0f + expf(-g));
  return g * sigmoid * u;
}
// sqrt(2/π) as the f64 product FRAC_2_SQRT_PI·FRAC_1_SQRT_2 rounded to f32.
constexpr float GLUE_SQRT_2_OVER_PI = (float)(1.12837916709551257390 * 0.70710678118654752440);
__device__ __forceinline__ float glue_gelu_mul(float g, float u) {
#pragma clang fp contract(off)
  const float inner = (g + g * g * g * 0.044715f) * GLUE_SQRT_2_OVER_PI;
  return ((g * (tanhf(inner) + 1.0f)) * 0.5f) * u;
}

}  // namespace

template <int OP, int DT, bool VEC>
__global__ __launch_bounds__(256) void glue_kernel(const void *__restrict__ a,
                                                   const void *__restrict__ b,
                                                   void *__restrict__ out, int64_t n) {
  constexpr int V = VEC ? (DT == RK_DTYPE_F32 ? 4 : 8) : 1;  // elements per thread
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * V;
  for (int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V; i0 < n; i0 += stride) {
    if (VEC && i0 + V <= n) {
      // 16-byte loads and store; elements in registers as f32
      const uintx4 av = *(const uintx4 *)((const uint8_t *)a + i0 * (16 / V));
      const uintx4 bv = *(const uintx4 *)((const uint8_t *)b + i0 * (16 / V));
      uintx4 ov;
      if constexpr (DT == RK_DTYPE_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = __uint_as_float(av[e]), u = __uint_as_float(bv[e]);
          ov[e] = __float_as_uint(OP == 0 ? glue_silu_mul(g, u) : glue_gelu_mul(g, u));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t w = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint16_t ga = (uint16_t)(av[e] >> (16 * h)), ub = (uint16_t)(bv[e] >> (16 * h));
            float g, u;
            if constexpr (DT == RK_DTYPE_F16) {
              g = (float)__builtin_bit_cast(f16, ga);
              u = (float)__builtin_bit_cast(f16, ub);
            } else {
              g = __uint_as_float((uint32_t)ga << 16);
              u = __uint_as_float((uint32_t)ub << 16);
            }
            const float r = OP == 0 ? glue_silu_mul(g, u) : glue_gelu_mul(g, u);
            const uint16_t rb = dt_encode<DT>(r);
            w |= (uint32_t)rb << (16 * h);
          }
          ov[e] = w;
        }
      }
      *(uintx4 *)((uint8_t *)out + i0 * (16 / V)) = ov;
    } else {
      for (int64_t i = i0; i < n && i < i0 + V; ++i) {
        const float g = dt_load<DT>(a, i), u = dt_load<DT>(b, i);
        dt_store<DT>(out, i, OP == 0 ? glue_silu_mul(g, u) : glue_gelu_mul(g, u));
      }
    }
  }
}

template <int OP, int DT>
static hipError_t launch_glue_t(const void *a, const void *b, void *out, int64_t n, hipStream_t st) {
  const bool vec = (((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) & 15) == 0;
  const int V = vec ? (DT == RK_DTYPE_F32 ? 4 : 8) : 1;
  const int64_t chunks = (n + V - 1) / V;
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 8192);
  if (vec)
    hipLaunchKernelGGL((glue_kernel<OP, DT, true>), dim3(blocks), dim3(256), 0, st, a, b, out, n);
  else
    hipLaunchKernelGGL((glue_kernel<OP, DT, false>), dim3(blocks), dim3(256), 0, st, a, b, out, n);
  return hipGetLastError();
}

hipError_t rk_launch_glue(int op, const void *a, const void *b, void *out, int64_t n, int dtype,
                          hipStream_t st) {
  if (n <= 0) return hipSuccess;
  switch (op * 3 + dtype) {
    case 0: return launch_glue_t<0, RK_DTYPE_F32>(a, b, out, n, st);
    case 1: return launch_glue_t<0, RK_DTYPE_F16>(a, b, out, n, st);
    case 2: return launch_glue_t<0, RK_DTYPE_BF16>(a, b, out, n, st);
    case 3: return launch_glue_t<1, RK_DTYPE_F32>(a, b, out, n, st);
    case 4: return launch_glue_t<1, RK_DTYPE_F16>(a, b, out, n, st);
    case 5: return launch_glue_t<1, RK_DTYPE_BF16>(a, b, out, n, st);
  }
  return hipErrorInvalidValue;
}
