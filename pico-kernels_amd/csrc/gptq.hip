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

// The same sweep for scale domains of at most 128 rows (group-wise GPTQ), with the block's
// values in registers: wave w of 16 holds columns 8w .. 8w + 7 of every row, lane l rows l and
// l + 64. A column's max is then one wave's (DPP, no barrier). Wave w first takes, column by
// column in order, the errors of every column before its own: it waits for the column's flag,
// reads the errors of its rows from LDS and applies them to its eight columns. Then it sweeps
// its own columns in registers: quantize, write the errors to LDS and raise the flag, apply
// them to its remaining columns. So every value still takes its updates in column order, the
// product rounded before the subtraction: bitwise the sweep above. The serial path is one
// flag hand-off between waves per eight columns instead of two workgroup barriers per column.
constexpr int kGptqFastRows = 128;
constexpr int kGptqFastCols = 128;
constexpr int kGptqFastWaves = 16;

__global__ __launch_bounds__(64 * kGptqFastWaves) void gptq_block_fast_kernel(GptqParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float lds[];
  float* rt = lds;                          // [nb][nb]: rt[c][c'] = ratio[b0 + c][b0 + c']
  float* eb = lds + p.nb * p.nb;            // [nb][128]: column c's errors by row
  __shared__ int ready[kGptqFastCols];      // ready[c] != 0: eb[c] is written
  constexpr int CPW = kGptqFastCols / kGptqFastWaves;  // columns per wave
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r0 = blockIdx.x * p.domain;
  const int rows = min(p.domain, p.out - r0);
  const int nb = p.nb;
  const int c0 = CPW * wave;  // this wave's first column

  {  // the ratios: every load in flight before the first LDS write
    constexpr int PER = kGptqFastCols * kGptqFastCols / (64 * kGptqFastWaves);
    float r[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = t + u * 64 * kGptqFastWaves, c = i / nb, c2 = i - c * nb;
      r[u] = i < nb * nb ? p.ratio[(int64_t)(p.b0 + c) * p.ldr + p.b0 + c2] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = t + u * 64 * kGptqFastWaves;
      if (i < nb * nb) rt[i] = r[u];
    }
  }
  if (t < kGptqFastCols) ready[t] = 0;
  bool live[2];
  float v[CPW][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) live[h] = lane + 64 * h < rows;
  {  // every load in flight at once: rows past the domain and columns past the block read a
     // valid element (row r0, column b0) and are never used
    const int64_t base = (int64_t)r0 * p.ldq + p.b0;
#pragma unroll
    for (int j = 0; j < CPW; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = c0 + j;
        const int64_t off = (live[h] ? (int64_t)(lane + 64 * h) * p.ldq : 0) + (c < nb ? c : 0);
        v[j][h] = p.q[base + off];
      }
  }
  __syncthreads();
  if (c0 >= nb) return;  // wave-uniform: no columns here

  // ---- the errors of every column before this wave's, in column order ----
  for (int c = 0; c < c0; ++c) {
    const float* rc = rt + c * nb;
    float r[CPW];  // read before the wait: the ratios do not change
#pragma unroll
    for (int j = 0; j < CPW; ++j) r[j] = rc[min(c0 + j, nb - 1)];
    // the owner runs in the same workgroup, so it is resident and the wait ends; the bound
    // only guards against a fault in that reasoning
    for (int i = 0; i < (1 << 26); ++i) {
      if (__hip_atomic_load(&ready[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");  // the error reads stay after the flag's
    float e[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) e[h] = eb[c * kGptqFastRows + lane + 64 * h];  // rows past: unused
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (c0 + j < nb) {  // wave-uniform
#pragma unroll
        for (int h = 0; h < 2; ++h) v[j][h] = v[j][h] - e[h] * r[j];
      }
    }
  }
  // this wave's own block of ratios, in registers for the serial part
  float ro[CPW][CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j)
#pragma unroll
    for (int j2 = 0; j2 < CPW; ++j2)
      ro[j][j2] = j2 > j ? rt[min(c0 + j, nb - 1) * nb + min(c0 + j2, nb - 1)] : 0.0f;

  // ---- this wave's own columns (their codes and errors kept in registers, stored at the end) ----
  const float fq = (float)p.qmax;
  float ev[CPW][2];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = c0 + j;
    ev[j][0] = ev[j][1] = 0.0f;
    if (c >= nb) continue;  // wave-uniform
    unsigned amax = 0u;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (live[h]) amax = max(amax, abs_bits(v[j][h]));
    const float a = __builtin_bit_cast(float, wave_max_u32(amax));
    const float s = (a < 1e-12f ? 1e-12f : a) / fq;  // clamp_min: NaN passes through
    float e[2], qv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float r = clamp_nan(__builtin_rintf(v[j][h] / s), -fq, fq);
      qv[h] = r * s;
      e[h] = v[j][h] - qv[h];
      if (live[h]) eb[c * kGptqFastRows + lane + 64 * h] = e[h];
    }
    // The errors land in LDS before the flag: lgkmcnt(0) orders this wave's LDS writes (a
    // release fence would also wait for global stores; there are none until the end).
    __builtin_amdgcn_s_waitcnt(0xc07f);
    if (lane == 0) __hip_atomic_store(&ready[c], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
    for (int h = 0; h < 2; ++h) ev[j][h] = e[h];
#pragma unroll
    for (int j2 = j + 1; j2 < CPW; ++j2) {
      if (c0 + j2 < nb) {  // wave-uniform
#pragma unroll
        for (int h = 0; h < 2; ++h) v[j2][h] = v[j2][h] - e[h] * ro[j][j2];
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) v[j][h] = qv[h];  // the column's codes times its scale
  }
  // codes and errors of this wave's columns, row by row: 16-byte stores where aligned
  const int ncols = min(CPW, nb - c0);
  const bool vec = ncols == CPW && p.ldq % 4 == 0 && p.lde % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(p.q + p.b0 + c0) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(p.err + c0) & 15) == 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (!live[h]) continue;
    float* qrow = p.q + (int64_t)(r0 + lane + 64 * h) * p.ldq + p.b0 + c0;
    float* erow = p.err + (int64_t)(r0 + lane + 64 * h) * p.lde + c0;
    if (vec) {
#pragma unroll
      for (int j = 0; j < CPW; j += 4) {
        *reinterpret_cast<pk_f4*>(qrow + j) = pk_f4{v[j][h], v[j + 1][h], v[j + 2][h], v[j + 3][h]};
        *reinterpret_cast<pk_f4*>(erow + j) = pk_f4{ev[j][h], ev[j + 1][h], ev[j + 2][h], ev[j + 3][h]};
      }
    } else {
#pragma unroll
      for (int j = 0; j < CPW; ++j)
        if (j < ncols) qrow[j] = v[j][h], erow[j] = ev[j][h];
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
  const int grid = (out + domain - 1) / domain;
  if (domain <= kGptqFastRows && nb <= kGptqFastCols) {
    const size_t lds = ((size_t)nb * nb + (size_t)nb * kGptqFastRows) * sizeof(float);
    static std::atomic<uint64_t> lds_fast{0};
    if (const int rc = set_lds_limit_once((const void*)gptq_block_fast_kernel, (int)(kGptqLdsFloats * sizeof(float)), &lds_fast)) return rc;
    gptq_block_fast_kernel<<<grid, 64 * kGptqFastWaves, lds, (hipStream_t)stream>>>(p);
    PK_LAUNCH_CHECK("gptq block");
    return PK_OK;
  }
  const size_t lds = ((size_t)nb * nb + (size_t)nb * domain) * sizeof(float);
  static std::atomic<uint64_t> lds_done{0};
  if (const int rc = set_lds_limit_once((const void*)gptq_block_kernel, (int)(kGptqLdsFloats * sizeof(float)), &lds_done)) return rc;
  gptq_block_kernel<<<grid, kGptqThreads, lds, (hipStream_t)stream>>>(p);
  PK_LAUNCH_CHECK("gptq block");
  return PK_OK;
}
