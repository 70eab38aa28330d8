// Fixed-order split-K reduction shared by the GEMV and the MFMA GEMM:
//   C[m, n] = scale * (((P[0][m][n] + P[1][m][n]) + P[2][m][n]) + ... + P[S-1][m][n]) (+ bias[n])
// where P is the (S, M, N) fp32 workspace written by the slices. Summing in slice order on
// the same element by the same thread makes the result independent of launch timing
// (the reference's split-K uses fp32 atomics instead, gemm_splitk.py:64).
#include "pk_internal.h"

#include <atomic>
#include <cstdlib>

namespace pk {

// The XCD grouping of xcd_tile_slice holds when the partition's XCC count divides 8 (SPX 8,
// DPX 4, QPX 2, CPX 1). Queried once per device.
int set_lds_limit_once(const void* kernel, int bytes, std::atomic<uint64_t>* done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "set LDS limit: hipGetDevice");
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done->load(std::memory_order_acquire) & bit)) return PK_OK;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return hip_status(e, "set LDS limit");
  if (bit) done->fetch_or(bit, std::memory_order_release);
  return PK_OK;
}

bool splitk_in_l2_ok() {
  static std::atomic<int> state[64];  // 0 unknown, 1 on, 2 off
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  int v = state[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    const char* env = std::getenv("PK_SPLITK_IN_L2");
    int nxcc = 0;
    const bool on = !(env && env[0] == '0') &&
                    hipDeviceGetAttribute(&nxcc, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess &&
                    (nxcc == 1 || nxcc == 2 || nxcc == 4 || nxcc == 8);
    v = on ? 1 : 2;
    state[dev].store(v, std::memory_order_relaxed);
  }
  return v == 1;
}

// One thread per 4 consecutive outputs; the S slice loads are unrolled so they are all in
// flight at once (the kernel is one memory round trip, not S of them). The four outputs go
// out as one 8-byte (fp16 / bf16) or 16-byte (fp32) store when `vec` (aligned rows).
template <int S, int DT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partials,
                                                            int M, int N, OutEpi epi,
                                                            void* __restrict__ c, bool vec,
                                                            int64_t ldc) {
  const int64_t plane4 = (int64_t)M * N / 4;  // N % 8 == 0, so rows hold whole quads
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= plane4) return;
  const pk_f4* src = reinterpret_cast<const pk_f4*>(partials) + q;
  pk_f4 part[S];
#pragma unroll
  for (int s = 0; s < S; ++s) part[s] = __builtin_nontemporal_load(src + s * plane4);
  pk_f4 v = part[0];
#pragma unroll
  for (int s = 1; s < S; ++s) v += part[s];
  const int64_t e = q * 4;
  const int64_t m = e / N, n = e - m * N;
  const int64_t o = m * ldc + n;
  store4_as<DT>(c, o, epi(v, n), vec);
}

// Generic slice count: the same fixed order. Loads go out in batches of 32 that are all in
// flight together, so S slices cost ceil(S / 32) memory round trips, not S.
constexpr int kReduceBatch = 32;
template <int DT>
__global__ __launch_bounds__(256) void splitk_reduce_any_kernel(const float* __restrict__ partials,
                                                                int S, int M, int N, OutEpi epi,
                                                                void* __restrict__ c, bool vec,
                                                                int64_t ldc) {
  const int64_t plane4 = (int64_t)M * N / 4;
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= plane4) return;
  const pk_f4* src = reinterpret_cast<const pk_f4*>(partials) + q;
  pk_f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < S; s0 += kReduceBatch) {
    pk_f4 part[kReduceBatch];
#pragma unroll
    for (int i = 0; i < kReduceBatch; ++i)
      if (s0 + i < S) part[i] = __builtin_nontemporal_load(src + (s0 + i) * plane4);
    // slice 0 starts the sum (so -0.0 partials stay -0.0, as in the fixed-S kernel)
    if (s0 == 0) v = part[0];
#pragma unroll
    for (int i = 0; i < kReduceBatch; ++i)
      if (s0 + i < S && s0 + i > 0) v += part[i];
  }
  const int64_t e = q * 4;
  const int64_t m = e / N, n = e - m * N;
  const int64_t o = m * ldc + n;
  store4_as<DT>(c, o, epi(v, n), vec);
}

int splitk_reduce(const float* partials, int S, int M, int N, OutEpi epi, void* c, int c_dtype,
                  int64_t ldc, hipStream_t s) {
  const int64_t quads = (int64_t)M * N / 4;
  const unsigned blocks = (unsigned)cdiv(quads, 256);
  const int esz = c_dtype == PK_F32 ? 4 : 2;
  const bool vec = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & (4 * esz - 1)) == 0;
  auto go = [&](auto DTC) {
    constexpr int dt = decltype(DTC)::value;
    switch (S) {
      case 2: splitk_reduce_kernel<2, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc); break;
      case 4: splitk_reduce_kernel<4, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc); break;
      case 8: splitk_reduce_kernel<8, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc); break;
      case 16: splitk_reduce_kernel<16, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc); break;
      case 32: splitk_reduce_kernel<32, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc); break;
      default:
        splitk_reduce_any_kernel<dt><<<blocks, 256, 0, s>>>(partials, S, M, N, epi, c, vec, ldc);
    }
  };
  if (c_dtype == PK_F32) go(pk_int_c<PK_F32>{});
  else if (c_dtype == PK_F16) go(pk_int_c<PK_F16>{});
  else go(pk_int_c<PK_BF16>{});
  PK_LAUNCH_CHECK("split-K reduce");
  return PK_OK;
}

}  // namespace pk
