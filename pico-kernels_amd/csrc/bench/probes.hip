// Ceiling probes for bench.py, built into their own library (libpk_bench_probes.so), outside
// the product library and its header; the reference has no counterpart:
//  * MFMA: waves that issue only independent MFMAs (no memory traffic in the loop), 8 waves
//    per workgroup like the GEMMs, on register operands that are either constant or
//    pseudo-random -- what the matrix cores sustain for the data the GEMMs see.
//  * HBM read: a streaming read of a buffer (16-byte non-temporal loads, XOR-reduced, one
//    word written per workgroup) -- what one launch reading a given number of bytes achieves,
//    the ceiling the memory-bound kernels' fractions are read against.
#include "../pk_common.h"

#include "pk_bench_probes.h"

namespace pk {

typedef int pk_i8v_probe __attribute__((ext_vector_type(8)));

// One LCG step per operand register; random operands keep magnitudes moderate (e4m3 bytes
// with the top exponent bit clear, fp16 values in [-1, 1]).
template <bool FP8, bool RAND>
__global__ __launch_bounds__(512) void mfma_probe_kernel(float* out, int iters) {
  const int t = threadIdx.x;
  unsigned s = (unsigned)t * 2654435761u ^ (unsigned)blockIdx.x * 40503u;
  pk_f16v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = (pk_f16v){};
  if constexpr (FP8) {
    pk_i8v_probe a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s = s * 1664525u + 1013904223u;
      a[i] = RAND ? (int)(s & 0x77777777u) : 0x38383838;
      s = s * 1664525u + 1013904223u;
      b[i] = RAND ? (int)(s & 0x77777777u) : 0x38383838;
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i], 0, 0, 0, 0, 0, 0);
    }
  } else {
    pk_half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s = s * 1664525u + 1013904223u;
      a[i] = RAND ? (pk_half)((float)((int)(s % 2001u) - 1000) * 0.001f) : (pk_half)0.5f;
      s = s * 1664525u + 1013904223u;
      b[i] = RAND ? (pk_half)((float)((int)(s % 2001u) - 1000) * 0.001f) : (pk_half)0.5f;
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
    }
  }
  float x = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) x += acc[i][r];
  out[(int64_t)blockIdx.x * 512 + t] = x;  // keeps the MFMAs live
}

// Grid-stride read of n16 16-byte words; each workgroup writes the XOR of what it read.
__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const pk_u4v* src, int64_t n16,
                                                             uint32_t* out) {
  uint32_t x = 0u;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {  // four loads in flight per thread
    const pk_u4v a = __builtin_nontemporal_load(src + i);
    const pk_u4v b = __builtin_nontemporal_load(src + i + stride);
    const pk_u4v c = __builtin_nontemporal_load(src + i + 2 * stride);
    const pk_u4v d = __builtin_nontemporal_load(src + i + 3 * stride);
    x ^= a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3] ^ c[0] ^ c[1] ^ c[2] ^ c[3] ^
         d[0] ^ d[1] ^ d[2] ^ d[3];
  }
  for (; i < n16; i += stride) {
    const pk_u4v a = __builtin_nontemporal_load(src + i);
    x ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  __shared__ uint32_t red[4];
  for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// The decode GEMV's read pattern with nothing else: one workgroup of 8 waves per 16-column
// strip (strip_bytes contiguous bytes, strips in the GEMV's XCD order), each wave loading its
// `u` consecutive 1 KB blocks with 16-byte non-temporal loads (lane L: bytes 16 L of each
// block), XOR-reducing them and writing one word per wave. No activations, scales, products or
// fold: the floor the strip GEMV's launch is read against.
__global__ __launch_bounds__(512) void strip_read_probe_kernel(const uint8_t* src, int strips,
                                                              int64_t strip_bytes, int u, int spx,
                                                              uint32_t* out) {
  const int s = (int)(blockIdx.x & 7) * spx + (int)(blockIdx.x >> 3);
  if (s >= strips) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src + (int64_t)s * strip_bytes, (uint32_t)strip_bytes);
  const int kb = (int)(strip_bytes / 1024);
  uint32_t x = 0u;
  for (int b0 = wave * u; b0 < kb; b0 += 8 * u) {
    pk_u4v v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = i < u && b0 + i < kb
                 ? __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, (b0 + i) * 1024, kPkLoadStream)
                 : pk_u4v{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  }
  for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
  if (lane == 0) out[blockIdx.x * 8 + wave] = x;
}

// The XCD (XCC id in the partition) each workgroup runs on. Each workgroup holds `lds_bytes`
// of dynamic LDS and sleeps about `spin` x 64 clocks before it records, so a grid larger
// than the machine is dispatched in several waves of residency, as the product's grids are.
__global__ void xcc_probe_kernel(uint32_t* out, int spin) {
  extern __shared__ uint32_t lds_hold[];
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  for (int i = 0; i < spin; ++i) __builtin_amdgcn_s_sleep(1);
  if (threadIdx.x == 0) {
    lds_hold[0] = v;
    out[blockIdx.x] = v & 0xfu;
  }
}

}  // namespace pk

using namespace pk;

extern "C" int pkb_xcc_count(void) {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) return -1;
  return n;
}

extern "C" int pkb_xcc_probe(int grid, int threads, int lds_bytes, int spin, uint32_t* out,
                             void* stream) {
  if (out == nullptr || grid < 1 || threads < 64 || threads > 1024 || threads % 64 ||
      lds_bytes < 4 || lds_bytes > 65536 || spin < 0 || spin > 100000)
    return -1;
  xcc_probe_kernel<<<grid, threads, lds_bytes, (hipStream_t)stream>>>(out, spin);
  return (int)hipGetLastError();
}

// Status: 0, or -1 for a bad argument, or the HIP error of the launch.
extern "C" int pkb_read_probe(const void* src, size_t bytes, uint32_t* out, int grid, void* stream) {
  if (src == nullptr || out == nullptr || grid < 1) return -1;
  if (bytes < 16 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15)) return -1;
  hbm_read_probe_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const pk_u4v*>(src), (int64_t)(bytes / 16), out);
  return (int)hipGetLastError();
}

extern "C" int pkb_strip_read_probe(const void* src, int strips, int64_t strip_bytes, int u,
                                    uint32_t* out, void* stream) {
  if (src == nullptr || out == nullptr || strips < 1 || strip_bytes < 1024 || strip_bytes % 1024 ||
      (u != 1 && u != 2 && u != 4 && u != 8) || (reinterpret_cast<uintptr_t>(src) & 15) ||
      strip_bytes >= (1ll << 31))
    return -1;
  const int spx = (strips + 7) / 8;
  strip_read_probe_kernel<<<8 * spx, 512, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const uint8_t*>(src), strips, strip_bytes, u, spx, out);
  return (int)hipGetLastError();
}

extern "C" int pkb_mfma_probe(int fp8, int random, int grid, int iters, float* out, void* stream) {
  if (out == nullptr || grid < 1 || iters < 1) return -1;
  const hipStream_t s = (hipStream_t)stream;
  if (fp8) {
    if (random) mfma_probe_kernel<true, true><<<grid, 512, 0, s>>>(out, iters);
    else mfma_probe_kernel<true, false><<<grid, 512, 0, s>>>(out, iters);
  } else {
    if (random) mfma_probe_kernel<false, true><<<grid, 512, 0, s>>>(out, iters);
    else mfma_probe_kernel<false, false><<<grid, 512, 0, s>>>(out, iters);
  }
  return (int)hipGetLastError();
}
