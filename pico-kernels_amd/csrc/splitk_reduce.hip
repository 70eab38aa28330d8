// Fixed-order split-K reduction shared by the GEMV and the MFMA GEMM:
//   C[m, n] = scale * (((P[0][m][n] + P[1][m][n]) + P[2][m][n]) + ... + P[S-1][m][n]) (+ bias[n])
// where P is the (S, M, N) fp32 workspace written by the slices. Summing in slice order on
// the same element by the same thread makes the result independent of launch timing
// (the reference's split-K uses fp32 atomics instead, gemm_splitk.py:64).
#include "pk_internal.h"

#include <atomic>
#include <cstdlib>
#include <mutex>

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

// The one-launch split-K forms hand partials off through one XCD's L2, which is right only
// while a launch's workgroup b runs on XCD (b + c) mod the partition's XCC count (c: where
// the launch starts). Before the first such launch on a device, a probe launch checks that
// rule on this machine: each of kPlacementGrid workgroups records its XCC id (hwreg XCC_ID)
// into a static device array (no allocation), the host copies it back on the caller's
// stream (one synchronisation of that stream, once per device) and checks every workgroup. A device that fails it (or whose XCC count does not divide 8,
// or with PK_SPLITK_IN_L2=0) uses the reduce launch instead: the same bits, one launch more.
constexpr int kPlacementGrid = 4096;
static __device__ __align__(256) uint32_t placement_xcc[kPlacementGrid];

__global__ __launch_bounds__(64) void xcd_placement_kernel(uint32_t* out) {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  if (threadIdx.x == 0) out[blockIdx.x] = v & 0xfu;
}

namespace {
std::atomic<int> g_l2_state[64];  // 0 not yet probed, 1 on, 2 off

int xcc_count(int dev) {
  int n = 0;
  return hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess ? n : 0;
}

bool l2_capable(int dev) {
  const char* env = std::getenv("PK_SPLITK_IN_L2");
  const int n = xcc_count(dev);
  return !(env && env[0] == '0') && (n == 1 || n == 2 || n == 4 || n == 8);
}

// Runs the probe on the current device, on the caller's stream (which it synchronises once):
// 1 when every workgroup obeyed the rule, 2 when one did not, 0 when the probe itself could
// not run (a HIP error: nothing is concluded).
int placement_probe(int nxcc, hipStream_t s) {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(placement_xcc)) != hipSuccess || ptr == nullptr)
    return 0;
  static uint32_t ids[kPlacementGrid];  // under the caller's first-use lock
  xcd_placement_kernel<<<kPlacementGrid, 64, 0, s>>>(static_cast<uint32_t*>(ptr));
  const bool ran = hipGetLastError() == hipSuccess &&
                   hipMemcpyAsync(ids, ptr, sizeof ids, hipMemcpyDeviceToHost, s) == hipSuccess &&
                   hipStreamSynchronize(s) == hipSuccess;
  if (!ran) return 0;
  const uint32_t c = ids[0];
  for (int b = 0; b < kPlacementGrid; ++b)
    if (ids[b] != (uint32_t)((b + c) % nxcc)) return 2;
  return 1;
}
}  // namespace

bool splitk_in_l2_possible() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  const int v = g_l2_state[dev].load(std::memory_order_acquire);
  return v == 0 ? l2_capable(dev) : v == 1;
}

bool splitk_in_l2_ok(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  int v = g_l2_state[dev].load(std::memory_order_acquire);
  if (v != 0) return v == 1;
  if (!l2_capable(dev)) {
    g_l2_state[dev].store(2, std::memory_order_release);
    return false;
  }
  // No probe (with its synchronisation) inside a stream capture: this call takes the reduce
  // launch, and the probe runs at the first call outside one.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (stream != nullptr && hipStreamIsCapturing(stream, &cap) != hipSuccess) return false;
  if (cap != hipStreamCaptureStatusNone) return false;
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  v = g_l2_state[dev].load(std::memory_order_acquire);
  if (v == 0) {
    v = placement_probe(xcc_count(dev), stream);
    if (v == 0) {  // the probe failed to run: the reduce launch this time, the probe again later
      (void)hipGetLastError();
      return false;
    }
    g_l2_state[dev].store(v, std::memory_order_release);
  }
  return v == 1;
}

// One thread per 4 consecutive outputs; the S slice loads are unrolled so they are all in
// flight at once (the kernel is one memory round trip, not S of them). The four outputs go
// out as one 8-byte (fp16 / bf16) or 16-byte (fp32) store when `vec` (aligned rows). TB
// threads per workgroup (256, or 64 after the register-dequant kernel: see splitk_reduce).
template <int S, int DT, int TB = 256>
__global__ __launch_bounds__(TB) void splitk_reduce_kernel(const float* __restrict__ partials,
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
                  int64_t ldc, hipStream_t s, bool small_groups) {
  const int64_t quads = (int64_t)M * N / 4;
  const bool g64 = small_groups && (S == 2 || S == 4 || S == 8);
  const unsigned blocks = (unsigned)cdiv(quads, g64 ? 64 : 256);
  const int esz = c_dtype == PK_F32 ? 4 : 2;
  const bool vec = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & (4 * esz - 1)) == 0;
  auto go = [&](auto DTC) {
    constexpr int dt = decltype(DTC)::value;
    switch (S) {
      case 2:
        if (g64) splitk_reduce_kernel<2, dt, 64><<<blocks, 64, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        else splitk_reduce_kernel<2, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        break;
      case 4:
        if (g64) splitk_reduce_kernel<4, dt, 64><<<blocks, 64, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        else splitk_reduce_kernel<4, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        break;
      case 8:
        if (g64) splitk_reduce_kernel<8, dt, 64><<<blocks, 64, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        else splitk_reduce_kernel<8, dt><<<blocks, 256, 0, s>>>(partials, M, N, epi, c, vec, ldc);
        break;
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
