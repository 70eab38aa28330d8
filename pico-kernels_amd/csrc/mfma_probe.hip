// Matrix-pipe ceiling probe: waves that issue only independent MFMAs (no memory traffic in
// the loop), 8 waves per workgroup like the GEMMs, on register operands that are either
// constant or pseudo-random. It measures what the matrix cores sustain on this GPU for the
// data the GEMMs see, the ceiling their roofline fractions are read against. A measurement
// entry point of this library; the reference has no counterpart.
#include "pk_internal.h"

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

}  // namespace pk

using namespace pk;

extern "C" int pk_mfma_probe(int fp8, int random, int grid, int iters, float* out, void* stream) {
  PK_REQUIRE(out != nullptr, "pk_mfma_probe: null output");
  PK_REQUIRE(grid >= 1 && iters >= 1, "pk_mfma_probe: grid and iters must be positive");
  const hipStream_t s = (hipStream_t)stream;
  if (fp8) {
    if (random) mfma_probe_kernel<true, true><<<grid, 512, 0, s>>>(out, iters);
    else mfma_probe_kernel<true, false><<<grid, 512, 0, s>>>(out, iters);
  } else {
    if (random) mfma_probe_kernel<false, true><<<grid, 512, 0, s>>>(out, iters);
    else mfma_probe_kernel<false, false><<<grid, 512, 0, s>>>(out, iters);
  }
  PK_LAUNCH_CHECK("mfma probe");
  return PK_OK;
}
