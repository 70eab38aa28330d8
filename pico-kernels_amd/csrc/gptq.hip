// GPTQ column sweep of one block of columns (the inner loop of the reference's gptq_layer,
// quantize.py:104-110), lazily batched: the caller applies the updates of earlier blocks with
// a GEMM, this kernel quantizes the block's columns one after another.
//
// Columns are swept in order. Quantizing column c uses its current value v (all updates from
// the block's earlier columns already applied), as quantize_col does (quantize.py:42-60):
// s = max|v over the scale domain|.clamp_min(1e-12) / qmax, q = clamp(rint(v / s), +-qmax) * s,
// e = v - q. Then every later column c' of the block takes v[c'] = v[c'] - e * ratio[c][c'],
// the product rounded before the subtraction: the reference's eager update
// `wq[:, j+1:] -= outer(err, ratio)` restricted to the block, so each column receives the same
// operations in the same order and the block's codes and errors equal the reference loop's bit
// for bit. The scale domain is a group of `group` consecutive rows, or the whole column.
//
// One workgroup of 1024 threads per scale domain: thread t owns row t % RT (RT = the domain's
// rows rounded up to a power of two, at most 1024; more rows are taken in strides of RT) and
// column group t / RT (CG = 1024 / RT groups). Group 0 quantizes and applies each column's
// errors to the next column; the other groups update the columns after that. The block's
// values (then, column by column, its errors) and ratios live in LDS; per column the threads
// meet twice: the max over the domain, the errors.
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

// |v| as an unsigned bit pattern: for non-negative floats and NaN these order the same way as
// the values (NaN above infinity), so maxima are branch-free integer maxima and a NaN wins
// as torch's max lets it.
__device__ __forceinline__ unsigned abs_bits(float v) { return __builtin_bit_cast(unsigned, v) & 0x7fffffffu; }

// Max over the wave: DPP within rows of 16 lanes, then the four rows.
__device__ __forceinline__ unsigned wave_max_u32(unsigned x) {
  int v = (int)x;
  auto mx = [](int a, int b) { return (unsigned)a > (unsigned)b ? a : b; };
  v = mx(v, __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, true));   // quad_perm [1,0,3,2]
  v = mx(v, __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, true));   // quad_perm [2,3,0,1]
  v = mx(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, true));  // row_half_mirror
  v = mx(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xf, 0xf, true));  // row_mirror
  return (unsigned)mx(mx(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
                      mx(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Workgroup barrier for LDS data only: this wave's LDS operations complete (lgkmcnt(0)), then
// s_barrier. Global stores stay in flight (__syncthreads() would wait for every one of them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}
constexpr int kGptqLdsFloats = 38 * 1024;  // 152 KiB of the 160 KiB LDS

__global__ __launch_bounds__(kGptqThreads) void gptq_block_kernel(GptqParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float lds[];
  float* rt = lds;                // [nb][nb]: rt[c][c'] = ratio[b0 + c][b0 + c']
  float* vh = lds + p.nb * p.nb;  // [nb][rows]: values, column c's errors once it is swept
  __shared__ __align__(16) unsigned red[kGptqThreads / 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r0 = blockIdx.x * p.domain;
  const int rows = min(p.domain, p.out - r0);
  const int nb = p.nb;
  int RT = 64;
  while (RT < rows && RT < kGptqThreads) RT <<= 1;
  const int CG = kGptqThreads / RT, lr0 = t % RT, cg = t / RT;

  for (int i = t; i < nb * nb; i += kGptqThreads) {
    const int c = i / nb, c2 = i - c * nb;
    rt[i] = p.ratio[(int64_t)(p.b0 + c) * p.ldr + p.b0 + c2];
  }
  for (int i = t; i < nb * rows; i += kGptqThreads) {  // row-contiguous global reads
    const int lr = i / nb, c = i - lr * nb;
    vh[c * rows + lr] = p.q[(int64_t)(r0 + lr) * p.ldq + p.b0 + c];
  }
  __syncthreads();

  const float fq = (float)p.qmax;
  for (int c = 0; c < nb; ++c) {
    float* vc = vh + c * rows;
    unsigned amax = 0u;
    if (cg == 0)
      for (int lr = lr0; lr < rows; lr += RT) amax = max(amax, abs_bits(vc[lr]));
    amax = wave_max_u32(amax);
    if (lane == 0) red[wave] = amax;
    lds_barrier();
    unsigned m4 = 0u;
#pragma unroll
    for (int w = 0; w < kGptqThreads / 64; w += 4) {  // all reads issued before any use
      const pk_u4v r4 = *reinterpret_cast<const pk_u4v*>(red + w);
      m4 = max(m4, max(max(r4[0], r4[1]), max(r4[2], r4[3])));
    }
    const float a = __builtin_bit_cast(float, m4);
    const float s = (a < 1e-12f ? 1e-12f : a) / fq;  // clamp_min: NaN passes through
    if (cg == 0) {
      for (int lr = lr0; lr < rows; lr += RT) {
        const float v = vc[lr];
        const float r = clamp_nan(__builtin_rintf(v / s), -fq, fq);
        const float qv = r * s;
        const float e = v - qv;
        vc[lr] = e;
        p.q[(int64_t)(r0 + lr) * p.ldq + p.b0 + c] = qv;
        p.err[(int64_t)(r0 + lr) * p.lde + c] = e;
      }
    }
    lds_barrier();  // column c's errors visible; every read of red done
    // Group 0 (the rows' quantizers) applies e to column c + 1 itself and goes on to quantize it;
    // the other groups update columns c + 2 .. and are waited for at the next column's first
    // barrier, before column c + 2 is read. A column's updates still arrive in column order.
    const float* rc = rt + c * nb;
    const int first = cg == 0 ? c + 1 : c + 2 + (cg - 1);
    const int stride = CG == 1 ? 1 : CG - 1;
    const int stop = (cg == 0 && CG > 1) ? min(c + 2, nb) : nb;
    for (int lr = lr0; lr < rows; lr += RT) {
      const float e = vc[lr];
      float* vr = vh + lr;
      int c2 = first;
      for (; c2 + 3 * stride < stop; c2 += 4 * stride) {  // all loads before any store (the
        float x[4], r[4];                                  // values and ratios share one array)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          x[u] = vr[(c2 + u * stride) * rows];
          r[u] = rc[c2 + u * stride];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) vr[(c2 + u * stride) * rows] = x[u] - e * r[u];
      }
      for (; c2 < stop; c2 += stride) vr[c2 * rows] = vr[c2 * rows] - e * rc[c2];
    }
  }
}

// Columns per block for a scale domain of `rows` rows: the largest power of two up to 128
// whose ratios and values fit the LDS budget; 0 if not even one column fits.
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
  static std::atomic<uint64_t> lds_done{0};
  if (const int rc = set_lds_limit_once((const void*)gptq_block_kernel, (int)(kGptqLdsFloats * sizeof(float)), &lds_done)) return rc;
  const int grid = (out + domain - 1) / domain;
  gptq_block_kernel<<<grid, kGptqThreads, lds, (hipStream_t)stream>>>(p);
  PK_LAUNCH_CHECK("gptq block");
  return PK_OK;
}
