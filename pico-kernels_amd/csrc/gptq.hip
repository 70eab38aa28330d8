// GPTQ column sweep of one block of columns (the inner loop of the reference's gptq_layer,
// quantize.py:104-110), lazily batched: the caller applies the updates of earlier blocks with
// a GEMM, this kernel quantizes the block's columns one after another.
//
// For column c of the block and every row r, the value to quantize is
//   v = Q[r, c] - sum_{j < c in the block} e[r, j] * ratio[j, c]
// with the terms subtracted in j order, each product rounded before its subtraction: the
// operations of the reference's eager update `wq[:, j+1:] -= outer(err, ratio)` applied to
// column c, in the same order. Then v is quantized as quantize_col does (quantize.py:42-60):
// s = max|v over the scale domain|.clamp_min(1e-12) / qmax, q = clamp(rint(v / s), +-qmax) * s,
// e = v - q. The scale domain is a group of `group` consecutive rows, or the whole column.
//
// One workgroup per scale domain. The block's ratios (transposed, rt[c][j]) and the domain's
// error history (e[j][row]) live in LDS; a thread owns rows t, t + T, ... of the domain. The
// only exchange between rows is the max per column (shuffles, then LDS across waves).
#include "pk_internal.h"

namespace pk {

struct GptqParams {
  float* q;            // [out, ldq] fp32, columns b0 .. b0 + nb - 1 swept in place
  int64_t ldq;
  const float* ratio;  // [in, ldr] fp32: ratio[j][c] = Hinv[j, c] / Hinv[j, j] for c > j
  int64_t ldr;
  float* err;          // [out, lde] fp32: err[r][c - b0] = e
  int64_t lde;
  int out, b0, nb, domain, qmax;
};

constexpr int kGptqThreads = 1024;
constexpr int kGptqLdsFloats = 38 * 1024;  // 152 KiB of the 160 KiB LDS

__global__ __launch_bounds__(kGptqThreads) void gptq_block_kernel(GptqParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float lds[];
  float* rt = lds;                          // [nb][nb]
  float* eh = lds + p.nb * p.nb;            // [nb][rows of the domain]
  __shared__ float red[kGptqThreads / 64];
  const int t = threadIdx.x, T = blockDim.x, lane = t & 63, wave = t >> 6, nw = T >> 6;
  const int r0 = blockIdx.x * p.domain;
  const int rows = min(p.domain, p.out - r0);
  const int nb = p.nb;

  for (int i = t; i < nb * nb; i += T) {
    const int c = i / nb, j = i - c * nb;
    rt[i] = j < c ? p.ratio[(int64_t)(p.b0 + j) * p.ldr + p.b0 + c] : 0.0f;
  }
  __syncthreads();

  const float fq = (float)p.qmax;
  for (int c = 0; c < nb; ++c) {
    const float* rc = rt + c * nb;
    float amax = 0.0f;
    for (int lr = t; lr < rows; lr += T) {
      float v = p.q[(int64_t)(r0 + lr) * p.ldq + p.b0 + c];
      int j = 0;
      for (; j + 4 <= c; j += 4) {
        const float e0 = eh[(j + 0) * rows + lr], e1 = eh[(j + 1) * rows + lr];
        const float e2 = eh[(j + 2) * rows + lr], e3 = eh[(j + 3) * rows + lr];
        v = v - e0 * rc[j + 0];
        v = v - e1 * rc[j + 1];
        v = v - e2 * rc[j + 2];
        v = v - e3 * rc[j + 3];
      }
      for (; j < c; ++j) v = v - eh[j * rows + lr] * rc[j];
      eh[c * rows + lr] = v;  // the value to quantize, until its error replaces it
      amax = nanmax(amax, __builtin_fabsf(v));
    }
    // max over the domain (order-free)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) amax = nanmax(amax, wave_shfl_xor(amax, m));
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float a = red[0];
    for (int w = 1; w < nw; ++w) a = nanmax(a, red[w]);
    __syncthreads();  // red is rewritten by the next column
    const float s = (a < 1e-12f ? 1e-12f : a) / fq;  // clamp_min: NaN passes through
    for (int lr = t; lr < rows; lr += T) {
      const float v = eh[c * rows + lr];
      const float r = clamp_nan(__builtin_rintf(v / s), -fq, fq);
      const float qv = r * s;
      const float e = v - qv;
      eh[c * rows + lr] = e;
      p.q[(int64_t)(r0 + lr) * p.ldq + p.b0 + c] = qv;
      p.err[(int64_t)(r0 + lr) * p.lde + c] = e;
    }
  }
}

// Columns per block for a scale domain of `rows` rows: the largest power of two up to 128
// whose ratios and error history fit the LDS budget; 0 if not even one column fits.
inline int gptq_block_cols(int rows) {
  for (int nb = 128; nb >= 1; nb >>= 1)
    if ((int64_t)nb * nb + (int64_t)nb * rows <= kGptqLdsFloats) return nb;
  return 0;
}

}  // namespace pk

using namespace pk;

extern "C" int pk_gptq_block_cols(int out, int group) {
  if (out < 1 || group < 0) return 0;
  const int domain = (group == 0 || group > out) ? out : group;
  return gptq_block_cols(domain);
}

extern "C" int pk_gptq_block(float* q, int64_t ldq, const float* ratio, int64_t ldr, float* err,
                             int64_t lde, int out, int in, int b0, int nb, int bits, int group,
                             void* stream) {
  PK_REQUIRE(q != nullptr && ratio != nullptr && err != nullptr, "pk_gptq_block: null pointer");
  PK_REQUIRE(out >= 1 && in >= 1, "pk_gptq_block: empty shape");
  PK_REQUIRE(bits >= 2 && bits <= 15, "pk_gptq_block: bits=%d must be in [2, 15]", bits);
  PK_REQUIRE(group >= 0, "pk_gptq_block: group=%d must be >= 0 (0: one scale per column)", group);
  PK_REQUIRE(b0 >= 0 && nb >= 1 && b0 + nb <= in, "pk_gptq_block: columns [%d, %d) outside [0, %d)",
             b0, b0 + nb, in);
  const int domain = (group == 0 || group > out) ? out : group;
  const int max_nb = gptq_block_cols(domain);
  PK_REQUIRE(max_nb >= 1, "pk_gptq_block: a scale domain of %d rows exceeds the LDS", domain);
  PK_REQUIRE(nb <= max_nb, "pk_gptq_block: nb=%d exceeds %d columns for a domain of %d rows", nb,
             max_nb, domain);
  PK_REQUIRE(ldq >= in && ldr >= in && lde >= nb, "pk_gptq_block: leading dimensions too small");
  GptqParams p;
  p.q = q;
  p.ldq = ldq;
  p.ratio = ratio;
  p.ldr = ldr;
  p.err = err;
  p.lde = lde;
  p.out = out;
  p.b0 = b0;
  p.nb = nb;
  p.domain = domain;
  p.qmax = (1 << (bits - 1)) - 1;
  const size_t lds = ((size_t)nb * nb + (size_t)nb * domain) * sizeof(float);
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute((const void*)gptq_block_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)(kGptqLdsFloats * sizeof(float)));
    if (e != hipSuccess) return hip_status(e, "gptq: set LDS size");
    attr_done = true;
  }
  const int threads = domain >= kGptqThreads ? kGptqThreads : ((domain + 63) / 64) * 64;
  const int grid = (out + domain - 1) / domain;
  gptq_block_kernel<<<grid, threads, lds, (hipStream_t)stream>>>(p);
  PK_LAUNCH_CHECK("gptq block");
  return PK_OK;
}
