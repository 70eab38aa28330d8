// Shared device/host helpers for the pico-kernels MI355X (gfx950) library.
//
// Everything here is written for CDNA4 only: 64-lane wavefronts, MFMA, 160 KB LDS.
// No CUDA-compat headers, no alternate code paths.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/pico_kernels_amd.h"

typedef _Float16 pk_half;
typedef _Float16 pk_half2 __attribute__((ext_vector_type(2)));
typedef _Float16 pk_half4 __attribute__((ext_vector_type(4)));
typedef _Float16 pk_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 pk_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pk_f4 __attribute__((ext_vector_type(4)));
typedef float pk_f16v __attribute__((ext_vector_type(16)));
typedef int pk_i8v __attribute__((ext_vector_type(8)));
typedef unsigned pk_u4v __attribute__((ext_vector_type(4)));
typedef unsigned pk_u2v __attribute__((ext_vector_type(2)));

constexpr unsigned kRsrcWord3 = 0x00020000u;  // raw (untyped) buffer, gfx9-family encoding

// Cache policy of a buffer load of data read exactly once (weights, K/V streams):
// non-temporal. Measured on MI355X: the M=1 GEMV 7-10% faster and split-KV decode attention 13%
// faster with their streams loaded this way (the bytes fetched from memory, FETCH_SIZE, are
// unchanged); it does not pay for the W4A16 kernel at 5 <= M <= 32 or for GEMM operands that
// several workgroups share.
constexpr int kPkLoadStream = 2;

// Raw buffer resource over [p, p + bytes): loads take a per-lane byte offset (VGPR) plus a
// wave-uniform one (SGPR), so row strides cost no vector instructions.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

// ---------------------------------------------------------------------------------------
// Error reporting (host side). Every C-ABI entry point returns PK_OK or a negative code and
// leaves a human-readable message retrievable with pk_last_error().
// ---------------------------------------------------------------------------------------
namespace pk {
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
}  // namespace pk

#define PK_REQUIRE(cond, ...)                      \
  do {                                             \
    if (!(cond)) {                                 \
      ::pk::set_error(__VA_ARGS__);                \
      return PK_EINVAL;                            \
    }                                              \
  } while (0)

#define PK_LAUNCH_CHECK(what) \
  do { hipError_t _e = hipGetLastError(); if (_e != hipSuccess) return ::pk::hip_status(_e, what); } while (0)

namespace pk {

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// Round-to-nearest-even float -> bf16 (NaN kept quiet). Used to reproduce bf16 tensor math.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Load element i of an fp32 / fp16 / bf16 array as float (exact widening).
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == PK_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == PK_F16) return (float)reinterpret_cast<const pk_half*>(p)[i];
  return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Round a float to the storage precision of `dtype` and back (what a torch op producing a
// tensor of that dtype does to its fp32 "opmath" result).
__device__ __forceinline__ float round_to_dtype(float v, int dtype) {
  if (dtype == PK_F16) return (float)(pk_half)v;  // v_cvt_f16_f32: round-to-nearest-even
  if (dtype == PK_BF16) return bf16_to_f32(f32_to_bf16_rne(v));
  return v;
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float v) {
  if (dtype == PK_F32) reinterpret_cast<float*>(p)[i] = v;
  else if (dtype == PK_F16) reinterpret_cast<pk_half*>(p)[i] = (pk_half)v;
  else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
}

// Output epilogue of the W4A16 matmuls: y[m, n] = scale * v (+ bias[n], a vector of N fp32 /
// fp16 / bf16 values, when one is given), rounded once to the output dtype by the store.
struct OutEpi {
  float scale;
  const void* bias;
  int bias_dtype;
  __host__ __device__ OutEpi(float s = 1.0f, const void* b = nullptr, int bd = PK_F16)
      : scale(s), bias(b), bias_dtype(bd) {}
  __device__ __forceinline__ float operator()(float v, int64_t n) const {
    v *= scale;
    if (bias != nullptr) v += load_as_f32(bias, bias_dtype, n);
    return v;
  }
  __device__ __forceinline__ pk_f4 operator()(pk_f4 v, int64_t n) const {
    v *= scale;
    if (bias != nullptr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += load_as_f32(bias, bias_dtype, n + e);
    }
    return v;
  }
};

// Waits out in-flight MFMAs before vector instructions read their accumulators. Measured on
// gfx950: when the last MFMA of an accumulation chain issues behind a predecessor that was
// itself issued late, the wait states the compiler counts from issue are not enough and an
// epilogue can read a partially written accumulator register. 128 wait states cover two
// back-to-back 16-pass MFMAs; the scheduling barriers keep everything on its side.
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile(
      "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Four consecutive outputs p[i .. i+3] of dtype DT: one 16-byte (fp32) or 8-byte (fp16/bf16)
// global store when `vec` (the caller has checked alignment), element stores otherwise.
#define PK_GLOBAL(T, ptr) ((__attribute__((address_space(1))) T*)(ptr))
template <int DT>
__device__ __forceinline__ void store4_as(void* p, int64_t i, pk_f4 v, bool vec) {
  if (!vec) {
#pragma unroll
    for (int e = 0; e < 4; ++e) store_from_f32(p, DT, i + e, v[e]);
    return;
  }
  if constexpr (DT == PK_F32) {
    *PK_GLOBAL(pk_f4, reinterpret_cast<float*>(p) + i) = v;
  } else if constexpr (DT == PK_F16) {
    const pk_half4 h = {(pk_half)v[0], (pk_half)v[1], (pk_half)v[2], (pk_half)v[3]};
    *PK_GLOBAL(pk_u2v, reinterpret_cast<pk_half*>(p) + i) = __builtin_bit_cast(pk_u2v, h);
  } else {
    const pk_u2v b = {(uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
                      (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16)};
    *PK_GLOBAL(pk_u2v, reinterpret_cast<uint16_t*>(p) + i) = b;
  }
}

// Calls f(std::integral_constant<int, DT>) for the runtime dtype, so loops inside f see a
// compile-time dtype.
template <int V>
struct pk_int_c {
  static constexpr int value = V;
};
template <typename F>
__device__ __forceinline__ void with_dtype(int dtype, F f) {
  if (dtype == PK_F32) f(pk_int_c<PK_F32>{});
  else if (dtype == PK_F16) f(pk_int_c<PK_F16>{});
  else f(pk_int_c<PK_BF16>{});
}

// OCP FP8 E4M3 ("e4m3fn": no infinities, S.1111.111 is NaN, max finite 448).
// Round-to-nearest-even, NOT saturating: any magnitude that rounds above 448 (that is,
// anything above 464, the tie point between 448 and the missing 480) and any Inf/NaN input
// becomes NaN (0x7f | sign). Written from the format definition:
//   normal:    (-1)^s * 2^(e-7) * (1 + m/8),   e in 1..15 (e=15,m=7 reserved for NaN)
//   subnormal: (-1)^s * 2^-6 * (m/8)
__host__ __device__ __forceinline__ uint8_t e4m3_from_f32(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x43e80000u) return sign | 0x7fu;           // > 464.0, Inf or NaN
  if (a < 0x3c800000u) {                              // below 2^-6: subnormal grid of 2^-9
    float mag = __builtin_bit_cast(float, a) * 512.0f;  // exact (power-of-two scaling)
    return sign | (uint8_t)__builtin_rintf(mag);      // 0..8; 8 is the smallest normal
  }
  // Normal range [2^-6, 464]: keep 3 mantissa bits with round-to-nearest-even. Adding
  // (half ulp - 1) plus the kept LSB then truncating is RNE; a mantissa carry correctly
  // bumps the exponent field.
  uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;  // = (f32 exp << 3) | mant3
  return sign | (uint8_t)(r - ((127u - 7u) << 3));
}

__host__ __device__ __forceinline__ float e4m3_to_f32(uint8_t v) {
  uint32_t s = (uint32_t)(v & 0x80u) << 24;
  uint32_t e = (v >> 3) & 15u, m = v & 7u;
  if (e == 15u && m == 7u) return __builtin_bit_cast(float, s | 0x7fc00000u);
  float mag;
  if (e == 0) mag = (float)m * (1.0f / 512.0f);
  else mag = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mag) | s);
}

// NaN-propagating max of non-negative values (torch's max propagates NaN).
__device__ __forceinline__ float nanmax(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// Clamp that propagates NaN the way torch.clamp does.
__device__ __forceinline__ float clamp_nan(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// ---------------------------------------------------------------------------------------
// Wave-level helpers (wave64).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// ---------------------------------------------------------------------------------------
// Split-K reduction inside one XCD's L2.
//
// MI355X dispatches the workgroups of a launch round-robin over its XCDs, each with its own
// L2: workgroup b goes to XCD (b + c) mod the partition's XCC count (8, 4, 2 or 1), the
// starting XCD c depending on earlier dispatches, so workgroups 8 ids apart share an XCD. A
// 1-D grid in which workgroup b takes column tile (b % 8) + 8 * ((b / 8) / split) and slice
// (b / 8) % split therefore keeps all slices of a tile on one XCD, whose L2 orders the
// handoff: each slice writes its fp32 partials (L1 is write-through) and waits for the
// stores to be acknowledged, then bumps the tile's arrival counter with an L2 atomic; the
// workgroup that arrives last adds the partials in slice order 0..split-1 -- the arithmetic
// of splitk_reduce_kernel, so the result is bitwise the same -- and resets the counter to 0
// for the next call. (Measured on MI355X: the partial lines are allocated in L2 by the
// stores without a fill, so the last workgroup's reads of them hit the tag but fetch the
// line from memory.) Grid slots past the last tile exit at once.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void xcd_tile_slice(int split, int& tile, int& slice) {
  const int b = blockIdx.x, jj = b >> 3;
  tile = (b & 7) + 8 * (jj / split);
  slice = jj % split;
}

// True, in every thread, for the last of the `split` workgroups that share *counter.
__device__ __forceinline__ bool splitk_arrive(unsigned* counter, int split) {
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are in L2
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const bool last = old == (unsigned)(split - 1);
    if (last) *counter = 0u;  // every slice has arrived: ready for the next call
    s_last = last;
  }
  __syncthreads();
  return s_last != 0;
}

// sum over s = 0..split-1 of p[s * stride] in slice order, `own_v` standing in for slice
// `own` (this workgroup's value); loads go out 16 at a time.
__device__ __forceinline__ float splitk_sum(const float* p, int64_t stride, int split, int own,
                                            float own_v) {
  float acc = 0.0f;
  for (int s0 = 0; s0 < split; s0 += 16) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (s0 + i < split) v[i] = (s0 + i == own) ? own_v : p[(int64_t)(s0 + i) * stride];
    if (s0 == 0) acc = v[0];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (s0 + i < split && s0 + i > 0) acc += v[i];
  }
  return acc;
}

}  // namespace pk
