// Per-tensor-scaled OCP e4m3 GEMM on the gfx950 fp8 matrix cores.
//
// C[M,N] = out_scale * (A8 @ B8), e4m3 inputs, fp32 accumulate on
// v_mfma_f32_16x16x128_f8f6f4 (both operands e4m3, unit block scales), the scale applied once
// in the epilogue (gemm_fp8.py:86) and the result stored as fp32 (the reference's dtype,
// gemm_fp8.py:107) or fp16/bf16.
//
// Layouts. A8 is (M, K) row-major. B8 is (K, N) row-major as in the reference
// (b_layout 0) or already transposed (N, K) (b_layout 1). The MFMA wants 32 consecutive k of
// one row (A) / one column (B) per lane, so both tiles live in LDS k-contiguous:
// As[BM][BK+16], Bs[BN][BK+16] bytes; the 16-byte pad keeps the 16-byte operand reads free
// of bank conflicts. For b_layout 0 each thread loads an 8(k) x 8(n) byte block and
// transposes it with byte permutes on the way into LDS.
//
// Tiling: 256 x 256 output tile, BK = 128, eight waves each owning 128 x 64 (8 x 4 MFMA
// fragments, 128 fp32 accumulators per lane), LDS double-buffered; 128 x 128 tiles with four
// waves for small problems.
#include "pk_internal.h"

namespace pk {

constexpr int kF8BK = 128;
constexpr int kF8Row = kF8BK + 16;  // bytes per LDS row

struct Fp8Params {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  int b_layout;
  float out_scale;
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ void f8_tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int total = tiles_m * tiles_n;
  int logical = bid;
  if (total % 8 == 0) logical = (bid % 8) * (total / 8) + bid / 8;
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_g = logical - g * per_group;
  *tm = first_m + in_g % gm;
  *tn = in_g / gm;
}

// 4x4 byte transpose: in[r] holds bytes (r, c=0..3); out[c] holds bytes (r=0..3, c).
__device__ __forceinline__ void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  const uint32_t t01a = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // r0c0 r1c0 r0c1 r1c1
  const uint32_t t01b = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // r0c2 r1c2 r0c3 r1c3
  const uint32_t t23a = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t t23b = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(t23a, t01a, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t23a, t01a, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t23b, t01b, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t23b, t01b, 0x07060302u);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int B_LAYOUT>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void fp8_gemm_kernel(Fp8Params p) {
  constexpr int T = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int A_ITEMS = BM * (kF8BK / 16);
  constexpr int A_PER_T = (A_ITEMS + T - 1) / T;
  constexpr int BT_ITEMS = BN * (kF8BK / 16);           // (N,K) layout: like A
  constexpr int BT_PER_T = (BT_ITEMS + T - 1) / T;
  constexpr int BN_ITEMS = (kF8BK / 8) * (BN / 8);      // (K,N) layout: 8k x 8n blocks
  constexpr int BN_PER_T = (BN_ITEMS + T - 1) / T;

  extern __shared__ __align__(16) char smem[];
  uint8_t* As = reinterpret_cast<uint8_t*>(smem);  // [2][BM][kF8Row]
  uint8_t* Bs = As + 2 * BM * kF8Row;              // [2][BN][kF8Row]

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  int tm, tn;
  f8_tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // K % 16 == 0 (checked on the host): the last tile may be partial; its 16-byte k chunks
  // past K (and, for (K, N) B, its 8-row groups past K) are zeroed like rows past M / N.
  const int ktiles = (p.K + kF8BK - 1) / kF8BK;

  uint4 areg[A_PER_T];
  uint4 btreg[B_LAYOUT == 1 ? BT_PER_T : 1];
  uint2 bnreg[B_LAYOUT == 0 ? BN_PER_T : 1][8];
  bool aok[A_PER_T], bok[B_LAYOUT == 1 ? BT_PER_T : BN_PER_T];

  // Loads are unconditional (addresses clamped into the matrix) so that no control flow
  // separates them from their use: the compiler can keep them in flight across the MFMAs
  // of the current tile. Out-of-range rows are zeroed when the tile is written to LDS.
  auto load_tile = [&](int kt) {
    const int k0 = kt * kF8BK;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int idx = i * T + t;
      const int row = (idx >> 3) % BM, kc = idx & 7;
      aok[i] = idx < A_ITEMS && m0 + row < p.M && k0 + kc * 16 < p.K;
      const int gm = min(m0 + row, p.M - 1);
      areg[i] = *reinterpret_cast<const uint4*>(p.a + (int64_t)gm * p.lda + min(k0 + kc * 16, p.K - 16));
    }
    if constexpr (B_LAYOUT == 1) {
#pragma unroll
      for (int i = 0; i < BT_PER_T; ++i) {
        const int idx = i * T + t;
        const int row = (idx >> 3) % BN, kc = idx & 7;
        bok[i] = idx < BT_ITEMS && n0 + row < p.N && k0 + kc * 16 < p.K;
        const int gn = min(n0 + row, p.N - 1);
        btreg[i] = *reinterpret_cast<const uint4*>(p.b + (int64_t)gn * p.ldb + min(k0 + kc * 16, p.K - 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < BN_PER_T; ++i) {
        const int idx = i * T + t;
        const int rk = idx & 15, cn = (idx >> 4) % (BN / 8);
        bok[i] = idx < BN_ITEMS && n0 + cn * 8 < p.N && k0 + rk * 8 < p.K;
        const int gn = min(n0 + cn * 8, p.N - 8);
#pragma unroll
        for (int r = 0; r < 8; ++r)
          bnreg[i][r] = *reinterpret_cast<const uint2*>(p.b + (int64_t)min(k0 + rk * 8 + r, p.K - 1) * p.ldb + gn);
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint8_t* as = As + buf * BM * kF8Row;
    uint8_t* bs = Bs + buf * BN * kF8Row;
    const uint4 z4 = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int idx = i * T + t;
      if (idx < A_ITEMS)
        *reinterpret_cast<uint4*>(as + (idx >> 3) * kF8Row + (idx & 7) * 16) = aok[i] ? areg[i] : z4;
    }
    if constexpr (B_LAYOUT == 1) {
#pragma unroll
      for (int i = 0; i < BT_PER_T; ++i) {
        const int idx = i * T + t;
        if (idx < BT_ITEMS)
          *reinterpret_cast<uint4*>(bs + (idx >> 3) * kF8Row + (idx & 7) * 16) = bok[i] ? btreg[i] : z4;
      }
    } else {
#pragma unroll
      for (int i = 0; i < BN_PER_T; ++i) {
        const int idx = i * T + t;
        if (idx >= BN_ITEMS) continue;
        const int rk = idx & 15, cn = idx >> 4;
        uint32_t col[8][2];  // col[c][q]: rows 4q..4q+3 of column c
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          uint32_t lo[4] = {bnreg[i][4 * q].x, bnreg[i][4 * q + 1].x, bnreg[i][4 * q + 2].x, bnreg[i][4 * q + 3].x};
          uint32_t hi[4] = {bnreg[i][4 * q].y, bnreg[i][4 * q + 1].y, bnreg[i][4 * q + 2].y, bnreg[i][4 * q + 3].y};
          uint32_t tl[4], th[4];
          transpose4x4(lo, tl);
          transpose4x4(hi, th);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            col[c][q] = bok[i] ? tl[c] : 0u;
            col[c + 4][q] = bok[i] ? th[c] : 0u;
          }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          uint2 v = {col[c][0], col[c][1]};
          *reinterpret_cast<uint2*>(bs + (cn * 8 + c) * kF8Row + rk * 8) = v;
        }
      }
    }
  };

  pk_f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f4){0.f, 0.f, 0.f, 0.f};

  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 15, lk = (lane >> 4) * 32;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    // Always prefetch (the last step re-reads the last tile into the idle buffer) so the
    // loop body has no branches between the loads and their consumer.
    load_tile(min(kt + 1, ktiles - 1));
    const uint8_t* as = As + buf * BM * kF8Row;
    const uint8_t* bs = Bs + buf * BN * kF8Row;
    pk_i8v bf[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint8_t* src = bs + (wn0 + 16 * j + lrow) * kF8Row + lk;
      uint4 x0 = *reinterpret_cast<const uint4*>(src);
      uint4 x1 = *reinterpret_cast<const uint4*>(src + 16);
      bf[j] = (pk_i8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const uint8_t* src = as + (wm0 + 16 * i + lrow) * kF8Row + lk;
      uint4 x0 = *reinterpret_cast<const uint4*>(src);
      uint4 x1 = *reinterpret_cast<const uint4*>(src + 16);
      const pk_i8v af = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], acc[i][j], 0, 0, 0, 0, 0, 0);
    }
    store_tile(buf ^ 1);
    __syncthreads();
  }
  mfma_drain();

  const int erow = 4 * (lane >> 4), ecol = lane & 15;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gm = m0 + wm0 + 16 * i + erow + r, gn = n0 + wn0 + 16 * j + ecol;
        if (gm < p.M && gn < p.N)
          store_from_f32(p.c, p.c_dtype, (int64_t)gm * p.ldc + gn, acc[i][j][r] * p.out_scale);
      }
}

template <int BM, int BN, int WMW, int WNW, int BL>
static int fp8_launch_cfg(Fp8Params& p, hipStream_t s) {
  constexpr size_t lds = (size_t)2 * (BM + BN) * kF8Row;
  static std::atomic<uint64_t> lds_done{0};
  if (const int rc = set_lds_limit_once((const void*)fp8_gemm_kernel<BM, BN, WMW, WNW, BL>, (int)lds, &lds_done)) return rc;
  p.tiles_m = (int)cdiv(p.M, BM);
  p.tiles_n = (int)cdiv(p.N, BN);
  fp8_gemm_kernel<BM, BN, WMW, WNW, BL><<<p.tiles_m * p.tiles_n, 64 * WMW * WNW, lds, s>>>(p);
  PK_LAUNCH_CHECK("fp8 gemm");
  return PK_OK;
}

}  // namespace pk

using namespace pk;

extern "C" int pk_fp8_gemm(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb,
                           int b_layout, float out_scale, void* c, int c_dtype, int64_t ldc,
                           int M, int N, int K, void* stream) {
  PK_REQUIRE(a8 != nullptr && b8 != nullptr && c != nullptr, "pk_fp8_gemm: null pointer");
  PK_REQUIRE(M >= 1 && N >= 1 && K >= 1, "pk_fp8_gemm: empty shape");
  PK_REQUIRE(K % 16 == 0, "pk_fp8_gemm: K=%d must be a multiple of 16", K);
  PK_REQUIRE(b_layout == 0 || b_layout == 1, "pk_fp8_gemm: b_layout must be 0 or 1");
  PK_REQUIRE(c_dtype == PK_F32 || c_dtype == PK_F16 || c_dtype == PK_BF16, "pk_fp8_gemm: out dtype");
  PK_REQUIRE(lda >= K && lda % 16 == 0 && (reinterpret_cast<uintptr_t>(a8) & 15) == 0,
             "pk_fp8_gemm: A rows must be 16-byte aligned (lda=%lld)", (long long)lda);
  if (b_layout == 1)
    PK_REQUIRE(ldb >= K && ldb % 16 == 0 && (reinterpret_cast<uintptr_t>(b8) & 15) == 0,
               "pk_fp8_gemm: B rows must be 16-byte aligned (ldb=%lld)", (long long)ldb);
  else
    PK_REQUIRE(ldb >= N && ldb % 8 == 0 && N % 8 == 0 && (reinterpret_cast<uintptr_t>(b8) & 7) == 0,
               "pk_fp8_gemm: (K,N) B needs N %% 8 == 0 and 8-byte aligned rows");
  PK_REQUIRE(ldc >= N, "pk_fp8_gemm: ldc < N");
  Fp8Params p;
  p.a = a8;
  p.lda = lda;
  p.b = b8;
  p.ldb = ldb;
  p.b_layout = b_layout;
  p.out_scale = out_scale;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  hipStream_t s = (hipStream_t)stream;
  // Large-tile 32x32x64 kernel (buffer DMA, swizzled LDS) when its loaders fit the shape.
  const bool v2_ok = M >= 64 && N >= 64 && K % 128 == 0 && N % 16 == 0 && lda % 16 == 0 &&
                     ldb % 16 == 0 &&
                     (reinterpret_cast<uintptr_t>(b8) & 15) == 0 &&
                     (int64_t)M * lda < (1ll << 31) &&
                     (b_layout == 1 ? (int64_t)N * ldb : (int64_t)K * ldb) < (1ll << 31);
  // Large shapes: the 4-stage kernel (both B layouts through LDS DMA; (K, N) B is read with
  // transposing LDS loads). Smaller ones: the 2-stage kernel with 128 x 128 tiles.
  if (f8_v3_ok(M, N, K, lda, ldb, b_layout, b8))
    return f8_v3_launch(a8, lda, b8, ldb, b_layout, out_scale, c, c_dtype, ldc, M, N, K, s);
  if (v2_ok) return v2_f8_launch(a8, lda, b8, ldb, b_layout, out_scale, c, c_dtype, ldc, M, N, K, s);
  const bool big = (int64_t)M * N >= (int64_t)2048 * 2048;
  if (b_layout == 1)
    return big ? fp8_launch_cfg<256, 256, 2, 4, 1>(p, s) : fp8_launch_cfg<128, 128, 2, 2, 1>(p, s);
  return big ? fp8_launch_cfg<256, 256, 2, 4, 0>(p, s) : fp8_launch_cfg<128, 128, 2, 2, 0>(p, s);
}
