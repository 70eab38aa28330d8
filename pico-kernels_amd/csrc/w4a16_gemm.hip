// MFMA GEMM for W4A16 prefill / batched decode, and the dense fp16 split-K GEMM.
//
// C[M,N] = tensor_scale * A[M,K] (fp16) @ B[K,N] (+ bias[N]), fp32 accumulate on
// v_mfma_f32_16x16x32_f16, with B either
//   * packed int4 (pack_int4_n words, gemm_int4.py:65-72), dequantised while it is staged
//     into LDS: q (exact in fp16 via the 0x6400 exponent trick) times the fp16 group scale,
//     or q alone in per-tensor mode (the scale then goes to the epilogue, as the reference's
//     `c * scale` at gemm_int4.py:92), or
//   * dense fp16 (K, N) row-major (gemm_splitk.py:26-80), transposed 8x8 in registers.
//
// Data layout in LDS: A tile [BM][BK+8] and B tile [BN][BK+8] fp16, both k-contiguous, so a
// lane's MFMA operand (8 consecutive k of one row/column) is one 16-byte ds_read; the 8-half
// row padding makes those reads bank-conflict free. Double-buffered: global loads for tile
// t+1 are in flight while tile t is multiplied; one barrier per K step.
//
// Split-K: grid.y slices K into contiguous ranges; slices write fp32 partial tiles to the
// workspace and splitk_reduce_kernel sums them in slice order, so results are reproducible
// bit for bit (no floating-point atomics).
#include <cstdlib>

#include "pk_internal.h"

namespace pk {

constexpr int kBK = 64;
constexpr int kLdsPad = 8;
constexpr int kLdsRow = kBK + kLdsPad;  // halves per LDS row

enum BMode { kBDenseF16 = 0, kBInt4 = 1, kBDenseBF16 = 2 };  // B operand (A matches dense B)

struct GemmParams {
  const pk_half* a;
  int64_t lda;
  const void* b;  // uint32 words (int4) or fp16
  int64_t ldb;    // words (int4) or elements (fp16)
  const pk_half* scales;  // int4 group scales (K/G, N) or null
  int group;
  OutEpi epi;  // tensor scale and optional bias
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int split, k_slice;
  int tiles_m, tiles_n;
  float* partials;  // (split, M, N) fp32 when split > 1
};

__device__ __forceinline__ pk_half2 h2(uint32_t v) { return __builtin_bit_cast(pk_half2, v); }
__device__ __forceinline__ uint32_t u32(pk_half2 v) { return __builtin_bit_cast(uint32_t, v); }

// Map the linear workgroup id to an output tile. Consecutive ids are dispatched round-robin
// over the 8 XCDs; regroup them so each XCD works on a compact block of tiles (shared A rows
// and B columns stay in that XCD's L2), then walk tiles in GROUP_M-tall column bands.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
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

template <int BM, int BN, int WAVES_M, int WAVES_N, int BMODE>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_mfma_kernel(GemmParams p) {
  constexpr int T = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;  // 16x16 fragments per wave
  constexpr int A_ITEMS = BM * (kBK / 8);     // 16-byte chunks of the A tile
  constexpr int A_PER_T = (A_ITEMS + T - 1) / T;
  constexpr int B_ITEMS = (kBK / 8) * (BN / 8);  // 8 rows x 8 columns blocks
  constexpr int B_PER_T = (B_ITEMS + T - 1) / T;
  static_assert(BM % (16 * WAVES_M) == 0 && BN % (16 * WAVES_N) == 0, "tile shape");

  extern __shared__ __align__(16) char smem[];
  pk_half* As = reinterpret_cast<pk_half*>(smem);            // [2][BM][kLdsRow]
  pk_half* Bs = As + 2 * BM * kLdsRow;                        // [2][BN][kLdsRow]

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int slice = blockIdx.y;
  const int k_begin = slice * p.k_slice;
  const int k_end = min(k_begin + p.k_slice, p.K);
  const int ktiles = (k_end - k_begin + kBK - 1) / kBK;

  // ---------------- global -> register staging -------------------------------------------
  // Loads are unconditional, with addresses clamped into the matrices, so no control flow
  // separates them from their consumer and they stay in flight across the current tile's
  // MFMAs. Validity is recorded and applied when the tile is written to LDS.
  uint4 areg[A_PER_T];
  uint32_t breg[B_PER_T][8][4];  // int4: [..][row][0]; fp16: [..][row][0..3]
  uint4 sreg[B_PER_T];
  bool aok[A_PER_T], bok[B_PER_T];
  const bool has_gs = p.scales != nullptr;

  auto load_tile = [&](int kt) {
    const int k0 = k_begin + kt * kBK;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int idx = i * T + t;
      const int row = (idx >> 3) % BM, kc = idx & 7;
      const int gm = m0 + row, gk = k0 + kc * 8;
      aok[i] = idx < A_ITEMS && gm < p.M && gk < k_end;
      areg[i] = *reinterpret_cast<const uint4*>(p.a + (int64_t)min(gm, p.M - 1) * p.lda + min(gk, p.K - 8));
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int idx = i * T + t;
      const int rg = idx & 7, cg = (idx >> 3) % (BN / 8);
      const int gk = min(k0 + rg * 8, p.K - 8);
      const int gn = min(n0 + cg * 8, p.N - 8);
      bok[i] = idx < B_ITEMS && k0 + rg * 8 < k_end && n0 + cg * 8 < p.N;
      if (BMODE == kBInt4) {
        const uint32_t* wq = reinterpret_cast<const uint32_t*>(p.b) + (gn >> 3);
#pragma unroll
        for (int r = 0; r < 8; ++r) breg[i][r][0] = wq[(int64_t)(gk + r) * p.ldb];
        if (has_gs) sreg[i] = *reinterpret_cast<const uint4*>(p.scales + (int64_t)(gk / p.group) * p.N + gn);
      } else {
        const pk_half* bh = reinterpret_cast<const pk_half*>(p.b) + gn;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint4 v = *reinterpret_cast<const uint4*>(bh + (int64_t)(gk + r) * p.ldb);
          breg[i][r][0] = v.x; breg[i][r][1] = v.y; breg[i][r][2] = v.z; breg[i][r][3] = v.w;
        }
      }
    }
  };

  // ---------------- register -> LDS (dequantise / transpose B) ----------------------------
  auto store_tile = [&](int buf) {
    pk_half* as = As + buf * BM * kLdsRow;
    pk_half* bs = Bs + buf * BN * kLdsRow;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int idx = i * T + t;
      if (idx < A_ITEMS) {
        const int row = idx >> 3, kc = idx & 7;
        const uint4 z4 = {0u, 0u, 0u, 0u};
        *reinterpret_cast<uint4*>(as + row * kLdsRow + kc * 8) = aok[i] ? areg[i] : z4;
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int idx = i * T + t;
      if (idx >= B_ITEMS) continue;
      const int rg = idx & 7, cg = idx >> 3;
      if (BMODE == kBInt4) {
        uint32_t w[8];
        // invalid blocks decode as code 0 (raw nibble 0 -> u = 8 after the XOR)
#pragma unroll
        for (int r = 0; r < 8; ++r) w[r] = (bok[i] ? breg[i][r][0] : 0u) ^ 0x88888888u;
        const bool gs = has_gs;
        const uint32_t sw[4] = {sreg[i].x, sreg[i].y, sreg[i].z, sreg[i].w};
        const pk_half2 bias = {(pk_half)1032.0f, (pk_half)1032.0f};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
          uint32_t pr[4];
#pragma unroll
          for (int r2 = 0; r2 < 4; ++r2) pr[r2] = __builtin_amdgcn_perm(w[2 * r2 + 1], w[2 * r2], sel);
#pragma unroll
          for (int hsel = 0; hsel < 2; ++hsel) {
            const int col = 2 * b + hsel;
            pk_half2 sc2;
            if (gs) {
              const uint32_t sv = sw[col >> 1];
              const uint32_t s1 = (col & 1) ? (sv >> 16) : (sv & 0xffffu);
              sc2 = h2(s1 | (s1 << 16));
            }
            uint4 out;
            uint32_t o[4];
#pragma unroll
            for (int r2 = 0; r2 < 4; ++r2) {
              const uint32_t nib = hsel ? (pr[r2] >> 4) : pr[r2];
              pk_half2 q = h2((nib & 0x000f000fu) | 0x64006400u) - bias;  // exact codes
              if (gs) q = q * sc2;
              o[r2] = u32(q);
            }
            out.x = o[0]; out.y = o[1]; out.z = o[2]; out.w = o[3];
            *reinterpret_cast<uint4*>(bs + (cg * 8 + col) * kLdsRow + rg * 8) = out;
          }
        }
      } else {
        // 8x8 fp16 transpose: column c of the block = rows 0..7 of that column.
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
          uint32_t o[4];
#pragma unroll
          for (int r2 = 0; r2 < 4; ++r2)
            o[r2] = bok[i] ? __builtin_amdgcn_perm(breg[i][2 * r2 + 1][c >> 1], breg[i][2 * r2][c >> 1], sel) : 0u;
          uint4 out = {o[0], o[1], o[2], o[3]};
          *reinterpret_cast<uint4*>(bs + (cg * 8 + c) * kLdsRow + rg * 8) = out;
        }
      }
    }
  };

  pk_f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f4){0.f, 0.f, 0.f, 0.f};

  load_tile(0);  // ktiles >= 1: every slice holds at least 32 rows
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 15, lk = (lane >> 4) * 8;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    // Always prefetch (the last step re-reads the last tile into the idle buffer) so the
    // loop body has no branches between the loads and their consumer.
    load_tile(min(kt + 1, ktiles - 1));
    const pk_half* as = As + buf * BM * kLdsRow;
    const pk_half* bs = Bs + buf * BN * kLdsRow;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      pk_half8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const pk_half8*>(as + (wm0 + 16 * i + lrow) * kLdsRow + kk + lk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const pk_half8*>(bs + (wn0 + 16 * j + lrow) * kLdsRow + kk + lk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          if constexpr (BMODE == kBDenseBF16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(pk_bf16x8, af[i]), __builtin_bit_cast(pk_bf16x8, bf[j]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    store_tile(buf ^ 1);
    __syncthreads();
  }

  mfma_drain();
  // ---------------- epilogue --------------------------------------------------------------
  // Fragment (i, j), register r holds C[m0+wm0+16i+4*(lane/16)+r][n0+wn0+16j+lane%16].
  const int erow = 4 * (lane >> 4), ecol = lane & 15;
  if (p.split == 1) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int gm = m0 + wm0 + 16 * i + erow + r, gn = n0 + wn0 + 16 * j + ecol;
          if (gm < p.M && gn < p.N)
            store_from_f32(p.c, p.c_dtype, (int64_t)gm * p.ldc + gn, p.epi(acc[i][j][r], gn));
        }
    return;
  }
  float* part = p.partials + (int64_t)slice * p.M * p.N;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gm = m0 + wm0 + 16 * i + erow + r, gn = n0 + wn0 + 16 * j + ecol;
        if (gm < p.M && gn < p.N) part[(int64_t)gm * p.N + gn] = acc[i][j][r];
      }
}

// ---------------------------------------------------------------------------------------
// Configurations and planning
// ---------------------------------------------------------------------------------------
static const GemmCfg kCfg16 = {16, 256, 1, 4};
static const GemmCfg kCfg32 = {32, 256, 1, 4};
static const GemmCfg kCfg64 = {64, 256, 1, 4};
static const GemmCfg kCfg128 = {128, 128, 2, 2};  // large-tile kernel: 128 x 128, 4 waves
static const GemmCfg kCfg256 = {256, 128, 2, 2};  // large-tile kernel: 256 x 128, 4 waves

static GemmCfg pick_cfg(int M) {
  if (M <= 16) return kCfg16;
  if (M <= 32) return kCfg32;
  if (M < 64) return kCfg64;
  if (M <= 128) return kCfg128;
  return kCfg256;
}

bool gemm_plan(int M, int N, int K, int group, bool has_gs, int split_req, GemmPlan* out) {
  if (M < 1 || N % 8 || K % 32) return false;
  GemmCfg cfg = pick_cfg(M);
  const int tiles_m = (int)cdiv(M, cfg.bm), tiles_n = (int)cdiv(N, cfg.bn);
  auto ok = [&](int s) {
    if (s < 1 || K % s) return false;
    const int ks = K / s;
    if (ks % 32) return false;
    if (s > 1 && ks % kBK) return false;
    return true;
  };
  int split = 1;
  if (split_req > 0) {
    if (!ok(split_req)) return false;
    split = split_req;
  } else if (cfg.bm >= 128) {
    // Large tiles run one workgroup per CU: the most slices that still fit the 256 CUs in one
    // round (measured best on the Llama-3-8B shapes at M = 64..256), each >= 512 rows of K.
    const int tiles = tiles_m * tiles_n;
    for (int s = 2; s <= 16; s *= 2) {
      if (!ok(s) || K / s < 512 || tiles * s > 256) break;
      split = s;
    }
  } else {
    // Enough workgroups to cover the 256 CUs, while each slice keeps >= 512 rows of K.
    const int tiles = tiles_m * tiles_n;
    for (int s = 1; s <= 16; s *= 2) {
      if (!ok(s)) break;
      if (K / s < 512 && s > 1) break;
      split = s;
      if (tiles * s >= 256) break;
    }
  }
  *out = {cfg, split, K / split, tiles_m, tiles_n};
  return true;
}

size_t gemm_workspace_bytes(const GemmPlan& pl, int M, int N) {
  if (pl.split <= 1) return 0;
  return kWsCounterBytes + (size_t)pl.split * M * N * sizeof(float);
}

template <int BM, int BN, int WMW, int WNW, int BMODE>
static int launch_cfg(const GemmParams& p, hipStream_t s) {
  constexpr size_t lds = (size_t)2 * (BM + BN) * kLdsRow * sizeof(pk_half);
  static std::atomic<uint64_t> lds_done{0};
  if (const int rc = set_lds_limit_once((const void*)gemm_mfma_kernel<BM, BN, WMW, WNW, BMODE>, (int)lds, &lds_done)) return rc;
  dim3 grid(p.tiles_m * p.tiles_n, p.split);
  gemm_mfma_kernel<BM, BN, WMW, WNW, BMODE><<<grid, 64 * WMW * WNW, lds, s>>>(p);
  PK_LAUNCH_CHECK("gemm mfma");
  return PK_OK;
}

template <int BMODE>
static int launch_mode(const GemmPlan& pl, const GemmParams& p, hipStream_t s) {
  const GemmCfg& c = pl.cfg;
  if (c.bm == 16) return launch_cfg<16, 256, 1, 4, BMODE>(p, s);
  if (c.bm == 32) return launch_cfg<32, 256, 1, 4, BMODE>(p, s);
  if (c.bm == 64) return launch_cfg<64, 256, 1, 4, BMODE>(p, s);
  if (c.bm == 128) return launch_cfg<128, 128, 2, 2, BMODE>(p, s);
  return launch_cfg<256, 128, 2, 2, BMODE>(p, s);
}

int gemm_launch(const GemmPlan& pl, int bmode, const void* a, int64_t lda, const void* b,
                int64_t ldb, const void* scales, int group, OutEpi epi, void* c,
                int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only) {
  // 128/256-row tiles: the large-tile 32x32-MFMA kernel when its constraints hold.
  if (pl.cfg.bm >= 128 &&
      v2_f16_ok(M, N, K, pl.k_slice, group, scales != nullptr, lda, ldb, bmode == kBInt4))
    return v2_f16_launch(pl.cfg.bm, bmode == kBInt4 ? 0 : (bmode == kBDenseBF16 ? 2 : 1), a, lda, b, ldb, scales, group,
                         epi, c, c_dtype, ldc, M, N, K, pl.split, workspace, s,
                         partials_only);
  GemmParams p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.b = b;
  p.ldb = ldb;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = group > 0 ? group : K;
  p.epi = epi;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.split = pl.split;
  p.k_slice = pl.k_slice;
  p.tiles_m = pl.tiles_m;
  p.tiles_n = pl.tiles_n;
  p.partials = pl.split > 1 ? split_partials(workspace, partials_only) : nullptr;
  int rc = bmode == kBInt4        ? launch_mode<kBInt4>(pl, p, s)
           : bmode == kBDenseBF16 ? launch_mode<kBDenseBF16>(pl, p, s)
                                  : launch_mode<kBDenseF16>(pl, p, s);
  if (rc != PK_OK || pl.split <= 1 || partials_only) return rc;
  return splitk_reduce(p.partials, pl.split, M, N, epi, c, c_dtype, ldc, s);
}

}  // namespace pk
