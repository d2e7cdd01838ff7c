// Shared definitions for the gfx950 kernels and the engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "../../include/burn_rocket_amd.h"

typedef _Float16 f16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_ __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));
typedef unsigned int uintx4 __attribute__((ext_vector_type(4)));
typedef unsigned int uintx2 __attribute__((ext_vector_type(2)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

// s_waitcnt immediates for gfx9: vmcnt[3:0] in bits 3:0, expcnt in 6:4,
// lgkmcnt in 11:8, vmcnt[5:4] in 15:14. A field at its maximum means "do not
// wait on this counter".
#define WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n)&15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))
#define WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0x0f | (7 << 4) | (0 << 8) | (3 << 14))
#define WAIT_ALL0() __builtin_amdgcn_s_waitcnt(0)

// Workgroup barrier without a memory fence. The kernels wait on the exact
// counters they need (WAIT_VMCNT / WAIT_LGKMCNT0) before it; the empty asm
// statements keep the compiler from moving memory operations across it.
#define BARRIER()                          \
  do {                                     \
    asm volatile("" ::: "memory");         \
    __builtin_amdgcn_s_barrier();          \
    asm volatile("" ::: "memory");         \
  } while (0)

// 64 zero bytes: the source of global→LDS copies that fall past the end of K,
// so a ragged K tail contributes nothing. One copy per translation unit.
static __device__ __attribute__((aligned(16))) uint8_t g_zero_chunk[64];

// Asynchronous 16-byte global→LDS copy (global_load_lds_dwordx4). The LDS
// destination of lane i is lds_base + 16·i; lds_base must be wave-uniform.
__device__ __forceinline__ void dma16(const void *gsrc, void *lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, LDS_PTR(lds_base), 16, 0, 0);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Logical→physical block index so that consecutive logical tiles land on the
// same XCD (the dispatcher assigns workgroup b to XCD b % 8). Tiles that share
// operands then share that XCD's L2.
__device__ __forceinline__ int xcd_swizzle(int b, int nblocks) {
  const int nx = 8;
  if (nblocks % nx != 0) return b;
  return (b % nx) * (nblocks / nx) + b / nx;
}

// The same for any grid size: XCD x receives workgroups x, x+8, x+16, ...,
// which become one contiguous range of logical indices.
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  const int nx = 8, x = b % nx, q = nblocks / nx, r = nblocks % nx;
  return x * q + min(x, r) + b / nx;
}

// Logical tile index → (tile row, tile column). group_m <= 0: row-fastest
// over the whole grid. Otherwise tiles come in groups of group_m tile rows,
// row-fastest inside a group, so a run of consecutive tiles (one XCD's share)
// reads a few A row-blocks and a few B column-blocks instead of all of A.
__device__ __forceinline__ void tile_coords(int L, int tiles_m, int tiles_n, int group_m, int &tm,
                                            int &tn) {
  if (group_m <= 0 || group_m >= tiles_m) {
    tm = L % tiles_m;
    tn = L / tiles_m;
    return;
  }
  const int per_group = group_m * tiles_n;
  const int g = L / per_group;
  const int first_m = g * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int l = L - g * per_group;
  tm = first_m + l % gm;
  tn = l / gm;
}


// ---- buffer resources and compile-time loops ------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Raw buffer descriptor word 3 for gfx9: 32-bit data format, no swizzle.
constexpr int RSRC_WORD3 = 0x00020000;

// Buffer over [base, base + bytes); loads at offsets past the end return 0.
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, int64_t bytes) {
  const int64_t b = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)b, RSRC_WORD3);
}
// A byte offset that is past the end of every buffer (the load returns 0).
constexpr uint32_t OOB_OFFSET = 0x80000000u;
// 16-byte buffer→LDS copy: lane i lands at lds_base + 16·i.
__device__ __forceinline__ void bdma16(rsrc_t r, void *lds_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(lds_base), 16, voff, soff, 0, 0);
}
template <int V>
using ic = std::integral_constant<int, V>;
template <typename F, int... U>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, U...>) {
  (f(ic<U>{}), ...);
}
// f(ic<0>{}), ..., f(ic<N-1>{}) in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

static inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }


// ---- element types of the float ops (RK_DTYPE_*) -----------------------------
// f32 → bf16 bits, round to nearest even; a NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
template <int DT>
using dt_storage = std::conditional_t<DT == RK_DTYPE_F32, uint32_t, uint16_t>;
// Storage bits → f32 (the argument is a scalar: see dt_load_vec).
template <int DT>
__device__ __forceinline__ float dt_decode(dt_storage<DT> s) {
  if constexpr (DT == RK_DTYPE_F32) return __uint_as_float(s);
  else if constexpr (DT == RK_DTYPE_F16) return (float)__builtin_bit_cast(f16, s);
  else return __uint_as_float((uint32_t)s << 16);
}
// f32 → storage bits, rounded to nearest even. For fp16 the value is pinned in
// a register first: left alone, the compiler folds a multiply that produced v
// into the conversion (v_fma_mixlo_f16), which rounds the exact product once
// to fp16 where an f32 result converted to fp16 is rounded twice; the two
// differ next to fp16 rounding midpoints.
template <int DT>
__device__ __forceinline__ dt_storage<DT> dt_encode(float v) {
  if constexpr (DT == RK_DTYPE_F32) {
    return __float_as_uint(v);
  } else if constexpr (DT == RK_DTYPE_F16) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (f16)v);
  } else {
    return f32_to_bf16_rne(v);
  }
}
template <int DT>
__device__ __forceinline__ float dt_load(const void *p, int64_t i) {
  return dt_decode<DT>(((const dt_storage<DT> *)p)[i]);
}
template <int DT>
__device__ __forceinline__ void dt_store(void *p, int64_t i, float v) {
  ((dt_storage<DT> *)p)[i] = dt_encode<DT>(v);
}
// Element type known only at run time (a wave-uniform branch).
__device__ __forceinline__ float dt_load_any(const void *p, int64_t i, int dt) {
  if (dt == RK_DTYPE_F32) return dt_load<RK_DTYPE_F32>(p, i);
  if (dt == RK_DTYPE_F16) return dt_load<RK_DTYPE_F16>(p, i);
  return dt_load<RK_DTYPE_BF16>(p, i);
}
// N consecutive elements from element i in one access; p + i must be aligned
// to N elements. Each element is copied to a scalar before it is decoded:
// hipcc 7.2 miscompiles a bit cast applied directly to a vector subscript.
template <int DT, int N>
__device__ __forceinline__ void dt_load_vec(const void *p, int64_t i, float *f) {
  using S = dt_storage<DT>;
  if constexpr (N == 1) {
    f[0] = dt_decode<DT>(((const S *)p)[i]);
  } else {
    typedef S SV __attribute__((ext_vector_type(N)));
    const SV v = *(const SV *)((const S *)p + i);
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const S s = v[e];
      f[e] = dt_decode<DT>(s);
    }
  }
}
template <int DT, int N>
__device__ __forceinline__ void dt_store_vec(void *p, int64_t i, const float *f) {
  using S = dt_storage<DT>;
  if constexpr (N == 1) {
    ((S *)p)[i] = dt_encode<DT>(f[0]);
  } else {
    typedef S SV __attribute__((ext_vector_type(N)));
    SV v;
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = dt_encode<DT>(f[e]);
    *(SV *)((S *)p + i) = v;
  }
}

// N elements kept as their storage bits, packed in dwords (loaded now, decoded
// later): lets a kernel issue the loads of several rows before it computes on
// any of them without one register per 16-bit value.
template <int DT, int N>
struct dt_raw {
  static constexpr int BYTES = N * (DT == RK_DTYPE_F32 ? 4 : 2);
  static constexpr int WORDS = BYTES < 4 ? 1 : BYTES / 4;
  uint32_t w[WORDS];
};
template <int DT, int N>
__device__ __forceinline__ void dt_load_raw(const void *p, int64_t i, dt_raw<DT, N> &r) {
  constexpr int ES = DT == RK_DTYPE_F32 ? 4 : 2;
  constexpr int W = dt_raw<DT, N>::WORDS;
  const uint8_t *a = (const uint8_t *)p + i * ES;
  if constexpr (dt_raw<DT, N>::BYTES < 4) {
    r.w[0] = *(const uint16_t *)a;
  } else if constexpr (W == 1) {
    r.w[0] = *(const uint32_t *)a;
  } else {
    typedef uint32_t UV __attribute__((ext_vector_type(W)));
    const UV x = *(const UV *)a;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint32_t u = x[k];
      r.w[k] = u;
    }
  }
}
template <int DT, int N>
__device__ __forceinline__ void dt_decode_raw(const dt_raw<DT, N> &r, float *f) {
#pragma unroll
  for (int e = 0; e < N; ++e) {
    if constexpr (DT == RK_DTYPE_F32)
      f[e] = __uint_as_float(r.w[e]);
    else
      f[e] = dt_decode<DT>((uint16_t)(r.w[e / 2] >> (16 * (e & 1))));
  }
}
