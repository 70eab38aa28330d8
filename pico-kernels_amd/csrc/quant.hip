// Quantization, packing and cast kernels (HBM-bound elementwise / column-group work).
//
// Reference semantics (torch rounding chain) reproduced bit-exactly:
//   gemm_int4.quantize_int4   gemm_int4.py:58-62
//   gemm_int4.pack_int4_n     gemm_int4.py:65-72   (+ the unpack at gemm_int4.py:44-49)
//   quantize.quantize_col     quantize.py:42-60
//   quantize.rtn_layer        quantize.py:63-68
//   gemm_fp8.quantize         gemm_fp8.py:89-95
#include "pk_common.h"

namespace pk {

constexpr int kThreads = 256;
constexpr int kMaxAbsmaxBlocks = 1024;

static inline dim3 grid_for(int64_t work_items, int per_thread) {
  int64_t b = cdiv(cdiv(work_items, per_thread), kThreads);
  if (b < 1) b = 1;
  if (b > 65535LL * 8) b = 65535LL * 8;
  return dim3((unsigned)b);
}

// ---------------------------------------------------------------------------------------
// absmax: per-block partial maxima (pass 1) then one block folds them (pass 2). Max is
// order-independent, so the result is exact and reproducible.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float block_max(float v, float* red) {
  for (int m = 32; m >= 1; m >>= 1) v = nanmax(v, wave_shfl_xor(v, m));
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) v = nanmax(v, red[w]);
    red[0] = v;
  }
  __syncthreads();
  return red[0];
}

__global__ __launch_bounds__(kThreads) void absmax_partial_kernel(const void* __restrict__ x,
                                                                  int dtype, int64_t n,
                                                                  float* __restrict__ partial) {
  __shared__ float red[kThreads / 64];
  float m = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (dtype == PK_F32) {
    const float* p = reinterpret_cast<const float*>(x);
    for (; i < n; i += stride) m = nanmax(m, __builtin_fabsf(p[i]));
  } else {
    // 16-bit types: 8 elements per 16-byte load on the aligned bulk.
    const uint16_t* p = reinterpret_cast<const uint16_t*>(x);
    int64_t n8 = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) ? n / 8 : 0;
    const uint4* p8 = reinterpret_cast<const uint4*>(x);
    for (int64_t j = i; j < n8; j += stride) {
      uint4 v = p8[j];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint16_t lo = (uint16_t)(w[t] & 0xffff), hi = (uint16_t)(w[t] >> 16);
        float a, b;
        if (dtype == PK_F16) {
          a = (float)__builtin_bit_cast(pk_half, lo);
          b = (float)__builtin_bit_cast(pk_half, hi);
        } else {
          a = bf16_to_f32(lo);
          b = bf16_to_f32(hi);
        }
        m = nanmax(m, nanmax(__builtin_fabsf(a), __builtin_fabsf(b)));
      }
    }
    for (int64_t j = n8 * 8 + i; j < n; j += stride) {
      float a = dtype == PK_F16 ? (float)__builtin_bit_cast(pk_half, p[j]) : bf16_to_f32(p[j]);
      m = nanmax(m, __builtin_fabsf(a));
    }
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void absmax_final_kernel(const float* __restrict__ partial,
                                                                int nparts,
                                                                float* __restrict__ out) {
  __shared__ float red[kThreads / 64];
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = nanmax(m, partial[i]);
  m = block_max(m, red);
  if (threadIdx.x == 0) out[0] = m;
}

static int absmax_blocks(int64_t n) {
  int64_t b = cdiv(n, (int64_t)kThreads * 16);
  if (b < 1) b = 1;
  if (b > kMaxAbsmaxBlocks) b = kMaxAbsmaxBlocks;
  return (int)b;
}

// ---------------------------------------------------------------------------------------
// Per-tensor int4 codes (gemm_int4.py:60-61): q = int8(clamp(round(T(w / s)), -8, 7)).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void quantize_int4_kernel(const void* __restrict__ w,
                                                                 int dtype, int64_t n,
                                                                 float scale,
                                                                 int8_t* __restrict__ q) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = load_as_f32(w, dtype, i);
    float t = round_to_dtype(v / scale, dtype);  // IEEE fp32 division, then tensor dtype
    float r = clamp_nan(__builtin_rintf(t), -8.0f, 7.0f);
    q[i] = (r == r) ? (int8_t)(int)r : (int8_t)0;
  }
}

// ---------------------------------------------------------------------------------------
// Pack / unpack (gemm_int4.py:65-72, 44-49).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void pack_int4_kernel(const int8_t* __restrict__ q,
                                                             int64_t rows, int64_t cols,
                                                             int64_t ldq,
                                                             uint8_t* __restrict__ out) {
  const int64_t half = cols / 2, total = rows * half;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t r = i / half, j = i - r * half;
    const int8_t* row = q + r * ldq;
    uint32_t lo = (uint32_t)(uint8_t)row[2 * j] & 0xfu;
    uint32_t hi = (uint32_t)(uint8_t)row[2 * j + 1] & 0xfu;
    out[i] = (uint8_t)(lo | (hi << 4));
  }
}

__global__ __launch_bounds__(kThreads) void unpack_int4_kernel(const uint8_t* __restrict__ p,
                                                               int64_t rows, int64_t cols,
                                                               int8_t* __restrict__ q) {
  const int64_t half = cols / 2, total = rows * half;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint32_t b = p[i];
    int lo = (int)(b & 0xfu), hi = (int)(b >> 4);
    q[2 * i] = (int8_t)(lo >= 8 ? lo - 16 : lo);
    q[2 * i + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
  }
}

// ---------------------------------------------------------------------------------------
// Group RTN quantization along K (quantize.py:42-68).
//
// One thread owns CPT consecutive columns of one group of rows. Pass 1 takes the group
// absmax per column, pass 2 quantizes (the group re-read hits L1/L2). With CPT == 8 and
// bits == 4 the thread emits whole 32-bit words of the packed (K, N/8) layout.
// ---------------------------------------------------------------------------------------
template <int CPT>
__global__ __launch_bounds__(kThreads) void quantize_group_kernel(
    const void* __restrict__ w, int dtype, int64_t K, int64_t N, int64_t ldw, int qmax,
    int group, int half_math, uint32_t* __restrict__ qweight, void* __restrict__ scales,
    int scale_dtype, void* __restrict__ fake, int fake_dtype) {
  const int64_t nchunks = cdiv(N, CPT);
  const int64_t ngroups = cdiv(K, group);
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= nchunks * ngroups) return;
  const int64_t g = item / nchunks, chunk = item - g * nchunks;
  const int64_t n0 = chunk * CPT, k0 = g * group;
  const int64_t k1 = (k0 + group < K) ? k0 + group : K;
  // In fp16/bf16 tensor math the 1e-12 floor is itself rounded to the tensor dtype
  // (it underflows to 0 in fp16).
  const int mdt = half_math ? dtype : PK_F32;
  const float floor_v = round_to_dtype(1e-12f, mdt);
  const float fq = (float)qmax;

  float s[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) s[c] = 0.0f;
  for (int64_t k = k0; k < k1; ++k) {
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      if (n0 + c < N) s[c] = nanmax(s[c], __builtin_fabsf(load_as_f32(w, dtype, k * ldw + n0 + c)));
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    float a = s[c] < floor_v ? floor_v : s[c];  // clamp_min, NaN passes through
    s[c] = round_to_dtype(a / fq, mdt);
    if (scales != nullptr && n0 + c < N) store_from_f32(scales, scale_dtype, g * N + n0 + c, s[c]);
  }
  for (int64_t k = k0; k < k1; ++k) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      if (n0 + c >= N) continue;
      float v = load_as_f32(w, dtype, k * ldw + n0 + c);
      float t = round_to_dtype(v / s[c], mdt);
      float r = clamp_nan(__builtin_rintf(t), -fq, fq);
      if (fake != nullptr) {
        float f = round_to_dtype(r * s[c], mdt);
        store_from_f32(fake, fake_dtype, k * N + n0 + c, f);
      }
      int code = (r == r) ? (int)r : 0;
      word |= ((uint32_t)code & 0xfu) << (4 * c);
    }
    if (CPT == 8 && qweight != nullptr) qweight[k * (N / 8) + chunk] = word;
  }
}

// ---------------------------------------------------------------------------------------
// Scaled e4m3 cast (gemm_fp8.py:95): out = e4m3(T(x * scale)).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void cast_e4m3_kernel(const void* __restrict__ x,
                                                             int dtype, int64_t n, float scale,
                                                             uint8_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t n4 = n / 4;
  uint32_t* out4 = reinterpret_cast<uint32_t*>(out);
  const bool vec = (reinterpret_cast<uintptr_t>(out) & 3) == 0;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    for (int64_t j = i; j < n4; j += stride) {
      uint32_t word = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float v = round_to_dtype(load_as_f32(x, dtype, 4 * j + t) * scale, dtype);
        word |= (uint32_t)e4m3_from_f32(v) << (8 * t);
      }
      out4[j] = word;
    }
    i += n4 * 4;
  }
  for (; i < n; i += stride) {
    float v = round_to_dtype(load_as_f32(x, dtype, i) * scale, dtype);
    out[i] = e4m3_from_f32(v);
  }
}

static bool float_dtype(int d) { return d == PK_F32 || d == PK_F16 || d == PK_BF16; }

}  // namespace pk

using namespace pk;

extern "C" size_t pk_absmax_workspace_bytes(int64_t n) {
  return (size_t)absmax_blocks(n < 1 ? 1 : n) * sizeof(float);
}

extern "C" int pk_absmax(const void* x, int x_dtype, int64_t n, float* out_dev, void* workspace,
                         size_t workspace_bytes, void* stream) {
  PK_REQUIRE(x != nullptr && out_dev != nullptr, "pk_absmax: null pointer");
  PK_REQUIRE(float_dtype(x_dtype), "pk_absmax: unsupported dtype %d", x_dtype);
  PK_REQUIRE(n >= 1, "pk_absmax: empty input (max of an empty tensor is undefined)");
  int blocks = absmax_blocks(n);
  if (workspace == nullptr || workspace_bytes < (size_t)blocks * sizeof(float)) {
    set_error("pk_absmax: workspace of %zu bytes needed", (size_t)blocks * sizeof(float));
    return PK_EWORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  float* partial = reinterpret_cast<float*>(workspace);
  absmax_partial_kernel<<<blocks, kThreads, 0, s>>>(x, x_dtype, n, partial);
  absmax_final_kernel<<<1, kThreads, 0, s>>>(partial, blocks, out_dev);
  PK_LAUNCH_CHECK("pk_absmax");
  return PK_OK;
}

extern "C" int pk_quantize_int4(const void* w, int w_dtype, int64_t n, float scale, int8_t* q,
                                void* stream) {
  PK_REQUIRE(w != nullptr && q != nullptr, "pk_quantize_int4: null pointer");
  PK_REQUIRE(float_dtype(w_dtype), "pk_quantize_int4: unsupported dtype %d", w_dtype);
  if (n <= 0) return PK_OK;
  quantize_int4_kernel<<<grid_for(n, 4), kThreads, 0, (hipStream_t)stream>>>(w, w_dtype, n,
                                                                              scale, q);
  PK_LAUNCH_CHECK("pk_quantize_int4");
  return PK_OK;
}

extern "C" int pk_pack_int4(const int8_t* q, int64_t rows, int64_t cols, int64_t ldq,
                            uint8_t* packed, void* stream) {
  PK_REQUIRE(q != nullptr && packed != nullptr, "pk_pack_int4: null pointer");
  PK_REQUIRE(rows >= 0 && cols >= 0 && cols % 2 == 0, "pk_pack_int4: N must be even");
  PK_REQUIRE(ldq >= cols, "pk_pack_int4: ldq < cols");
  if (rows * cols == 0) return PK_OK;
  pack_int4_kernel<<<grid_for(rows * cols / 2, 4), kThreads, 0, (hipStream_t)stream>>>(
      q, rows, cols, ldq, packed);
  PK_LAUNCH_CHECK("pk_pack_int4");
  return PK_OK;
}

extern "C" int pk_unpack_int4(const uint8_t* packed, int64_t rows, int64_t cols, int8_t* q,
                              void* stream) {
  PK_REQUIRE(q != nullptr && packed != nullptr, "pk_unpack_int4: null pointer");
  PK_REQUIRE(rows >= 0 && cols >= 0 && cols % 2 == 0, "pk_unpack_int4: N must be even");
  if (rows * cols == 0) return PK_OK;
  unpack_int4_kernel<<<grid_for(rows * cols / 2, 4), kThreads, 0, (hipStream_t)stream>>>(
      packed, rows, cols, q);
  PK_LAUNCH_CHECK("pk_unpack_int4");
  return PK_OK;
}

extern "C" int pk_quantize_group(const void* w, int w_dtype, int64_t K, int64_t N, int64_t ldw,
                                 int bits, int group_size, int half_math, uint32_t* qweight,
                                 void* scales, int scale_dtype, void* fake, int fake_dtype,
                                 void* stream) {
  PK_REQUIRE(w != nullptr, "pk_quantize_group: null weight");
  PK_REQUIRE(float_dtype(w_dtype), "pk_quantize_group: unsupported dtype %d", w_dtype);
  PK_REQUIRE(K >= 0 && N >= 0 && ldw >= N, "pk_quantize_group: bad shape");
  PK_REQUIRE(bits >= 2 && bits <= 15, "pk_quantize_group: bits must be in [2, 15]");
  PK_REQUIRE(!half_math || w_dtype != PK_F32, "pk_quantize_group: half_math needs fp16/bf16");
  PK_REQUIRE(qweight == nullptr || (bits == 4 && N % 8 == 0),
             "pk_quantize_group: packed output needs bits == 4 and N % 8 == 0");
  PK_REQUIRE(scales == nullptr || float_dtype(scale_dtype), "pk_quantize_group: scale dtype");
  PK_REQUIRE(fake == nullptr || float_dtype(fake_dtype), "pk_quantize_group: fake dtype");
  if (K == 0 || N == 0) return PK_OK;
  const int group = group_size > 0 ? group_size : (int)K;
  const int qmax = (1 << (bits - 1)) - 1;
  hipStream_t s = (hipStream_t)stream;
  const int64_t groups = cdiv(K, group);
  if (qweight != nullptr || N % 8 == 0) {
    int64_t items = cdiv(N, 8) * groups;
    quantize_group_kernel<8><<<(unsigned)cdiv(items, kThreads), kThreads, 0, s>>>(
        w, w_dtype, K, N, ldw, qmax, group, half_math, qweight, scales, scale_dtype, fake,
        fake_dtype);
  } else {
    int64_t items = N * groups;
    quantize_group_kernel<1><<<(unsigned)cdiv(items, kThreads), kThreads, 0, s>>>(
        w, w_dtype, K, N, ldw, qmax, group, half_math, nullptr, scales, scale_dtype, fake,
        fake_dtype);
  }
  PK_LAUNCH_CHECK("pk_quantize_group");
  return PK_OK;
}

extern "C" int pk_cast_e4m3(const void* x, int x_dtype, int64_t n, float scale, uint8_t* out,
                            void* stream) {
  PK_REQUIRE(x != nullptr && out != nullptr, "pk_cast_e4m3: null pointer");
  PK_REQUIRE(float_dtype(x_dtype), "pk_cast_e4m3: unsupported dtype %d", x_dtype);
  if (n <= 0) return PK_OK;
  cast_e4m3_kernel<<<grid_for(n, 8), kThreads, 0, (hipStream_t)stream>>>(x, x_dtype, n, scale,
                                                                          out);
  PK_LAUNCH_CHECK("pk_cast_e4m3");
  return PK_OK;
}
