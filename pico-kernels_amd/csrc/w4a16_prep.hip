// Activation preparation for the W4A16 matmul of per-input-feature quantized weights.
//
// The reference's quantize_model (quantize.py:160-181) writes back, for every linear layer
// W [out, in], wq[:, j] = q[:, j] * s_j with ONE scale per input feature j taken over all
// output rows (quantize_col with group_size=None, quantize.py:52-54, through rtn_layer or
// gptq_layer, quantize.py:63-115). The product x @ wq^T = (x * s) @ q^T, so the packed layer
// keeps the int4 codes q^T (in, out) and folds s into the activations:
//   y[m, k] = fp16(x[m, k] * s[k] * mul)        (x fp32, fp16 or bf16; s fp32, optional)
// after which the W4A16 kernels run in their per-tensor mode with tensor_scale = 1 / mul.
// With s absent this is the input cast (fp32 / bf16 -> fp16) of the packed linear layer.
// One pass over x: 8 consecutive k per thread (K % 8 == 0), a 16-byte fp16 store.
#include "pk_internal.h"

namespace pk {

template <int XD, bool HAS_S>
__global__ __launch_bounds__(256) void w4a16_prep_kernel(const void* __restrict__ x, int64_t ldx,
                                                         const float* __restrict__ s, float mul,
                                                         pk_half* __restrict__ y, int64_t ldy,
                                                         int M, int K, int chunks) {
  const int m = blockIdx.x / chunks;  // one row per `chunks` workgroups of 2048 k
  const int k0 = ((blockIdx.x % chunks) * 256 + threadIdx.x) * 8;
  if (m >= M || k0 >= K) return;
  float v[8];
  if constexpr (XD == PK_F32) {
    const float* xr = reinterpret_cast<const float*>(x) + (int64_t)m * ldx + k0;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = xr[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = load_as_f32(x, XD, (int64_t)m * ldx + k0 + i);
  }
  pk_half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float t = v[i];
    if constexpr (HAS_S) t = t * s[k0 + i];
    h[i] = (pk_half)(t * mul);
  }
  *reinterpret_cast<pk_half8*>(y + (int64_t)m * ldy + k0) = h;
}

}  // namespace pk

using namespace pk;

extern "C" int pk_w4a16_prep_activations(const void* x, int x_dtype, int64_t ldx,
                                         const float* in_scale, float mul, void* y, int64_t ldy,
                                         int M, int K, void* stream) {
  PK_REQUIRE(x != nullptr && y != nullptr, "pk_w4a16_prep_activations: null pointer");
  PK_REQUIRE(M >= 1 && K >= 8 && K % 8 == 0, "pk_w4a16_prep_activations: M=%d K=%d (K %% 8)", M, K);
  PK_REQUIRE(x_dtype == PK_F32 || x_dtype == PK_F16 || x_dtype == PK_BF16,
             "pk_w4a16_prep_activations: input dtype %d", x_dtype);
  PK_REQUIRE(ldx >= K && ldy >= K && ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0,
             "pk_w4a16_prep_activations: output rows must be 16-byte aligned (ldy=%lld)",
             (long long)ldy);
  const hipStream_t s = (hipStream_t)stream;
  const int chunks = (int)cdiv(K / 8, 256);
  PK_REQUIRE((int64_t)chunks * M < (1ll << 31), "pk_w4a16_prep_activations: M=%d too large", M);
  const unsigned grid = (unsigned)(chunks * M);
  pk_half* yh = reinterpret_cast<pk_half*>(y);
  auto go = [&](auto DT) {
    constexpr int xd = decltype(DT)::value;
    if (in_scale) w4a16_prep_kernel<xd, true><<<grid, 256, 0, s>>>(x, ldx, in_scale, mul, yh, ldy, M, K, chunks);
    else w4a16_prep_kernel<xd, false><<<grid, 256, 0, s>>>(x, ldx, nullptr, mul, yh, ldy, M, K, chunks);
  };
  if (x_dtype == PK_F32) go(pk_int_c<PK_F32>{});
  else if (x_dtype == PK_F16) go(pk_int_c<PK_F16>{});
  else go(pk_int_c<PK_BF16>{});
  PK_LAUNCH_CHECK("w4a16 activation prep");
  return PK_OK;
}
