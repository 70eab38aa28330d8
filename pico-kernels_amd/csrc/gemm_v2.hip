// Large-tile MFMA GEMMs for gfx950: W4A16 / dense fp16 (v_mfma_f32_32x32x16_f16) and
// e4m3 fp8 (v_mfma_f32_32x32x64_f8f6f4).
//
// Design (f16: 8 waves, two per SIMD: 256 x 128 tiles as 4 x 2 waves of 64 x 64, 128 x 128
// tiles as 2 x 4 waves of 64 x 32; fp8 256 x 256: 8 waves, 2 x 4, each a 128 x 64 block):
//  * LDS tiles are rows of 128 bytes (64 fp16 or 128 fp8 values of k) in 8 chunks of 16 B;
//    chunk c of row r is stored in slot c ^ ((r >> 1) & 7). Sixteen lanes reading 16
//    consecutive rows at one chunk then touch 16 distinct 16-byte bank groups.
//  * A (and a (N, K) fp8 B) go global -> LDS by buffer DMA (buffer_load ... lds): no VGPR
//    staging, no ds_write. Each pipeline stage is its own __shared__ array so the compiler's
//    wait-count insertion only waits for DMA into the stage being read.
//  * int4 B is loaded into registers, dequantised (exact codes via the 0x6400 fp16 exponent
//    trick, times the fp16 group scale) and written k-contiguous; (K, N) fp16/fp8 B is
//    transposed with byte permutes on the same path.
//  * Pipelining: the loads of later tiles are issued before the MFMAs of tile t and
//    consumed after them (three stages for f16, two for fp8); one barrier per tile.
//  * Addresses: one buffer resource per operand, per-lane byte offsets computed once, the K
//    advance folded into the scalar offset. Rows/columns past the matrix are clamped to the
//    last valid one (never read out of bounds); their results are not stored.
//  * Epilogue (f16 kernel): each wave stages its block of C (or of the split-K partials) in a
//    free stage array and stores it back row-contiguous, whole 128-byte lines per store
//    instruction.
#include "pk_internal.h"

namespace pk {

#define PK_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// 16 bytes per lane, global -> LDS (lane L writes lds + 16 L). A device-only helper: the
// generic-to-LDS pointer cast must not appear in host-visible code (lambdas are host+device
// and the host pass would otherwise drop the kernel that uses them).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS(lds), 16, voff, soff, 0, 0);
}

// Byte offset of chunk c of row r in a swizzled 128-byte-row tile.
__device__ __forceinline__ int swz(int r, int c) { return (r << 7) + ((c ^ ((r >> 1) & 7)) << 4); }

__device__ __forceinline__ pk_half2 h2v(uint32_t v) { return __builtin_bit_cast(pk_half2, v); }
__device__ __forceinline__ uint32_t u32v(pk_half2 v) { return __builtin_bit_cast(uint32_t, v); }

// XCD-aware tile order (see w4a16_gemm.hip): regroup the round-robin XCD dispatch so each XCD
// owns a compact block of output tiles, then walk them GROUP_M tiles tall.
__device__ __forceinline__ void v2_tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
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

struct V2Params {
  const void* a;
  int64_t lda;            // elements
  const void* b;          // int4 words / fp16 / fp8
  int64_t ldb;            // words (int4) or elements
  const pk_half* scales;  // int4 group scales (K/G, N) or null
  int group;
  OutEpi epi;             // epilogue: tensor scale / fp8 out_scale, optional bias
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int split, k_slice;
  int tiles_m, tiles_n;
  float* partials;        // (split, M, N) when split > 1
};

enum V2B { kV2Int4 = 0, kV2F16KN = 1, kV2BF16KN = 2 };  // B (K, N): int4 words, fp16, bf16

// ---------------------------------------------------------------------------------------
// 3-stage f16 MFMA kernel, BM x 128 tiles (A fp16 (M, K); B int4 words or fp16 (K, N));
// BK = 64, 4 waves (2 x 2).
//
// Swapped MFMA operands (B first) make each accumulator C^T, so a lane holds four consecutive
// output columns per register quad (8- or 16-byte stores). Three LDS stages: the A DMA of
// tile t+2 and the B words of tile t+2 issued after the barrier of tile t, and the B words of
// tile t+1 dequantised into their stage while tile t is multiplied. Per tile one bare
// s_barrier: __syncthreads() would
// add a release fence that waits for every outstanding LDS DMA and undo the prefetch; the
// explicit wait before the barrier (this wave's DMA of tile t and its ds_writes of tile t's
// B) publishes exactly what the next step reads.
// ---------------------------------------------------------------------------------------
// NWM x NWN waves, two per SIMD (measured on MI355X: one wave per SIMD reads LDS at ~96 B/clk
// per CU, two at ~170): BM = 256 as 4 x 2 waves of 64 x 64; BM = 128 as 2 x 4 waves of 64 x 32
// for M <= 128, where 256-row tiles would leave half the MFMA work on padding rows.
template <int BMODE, bool GS, int BM, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN)
__attribute__((amdgpu_waves_per_eu(NWM * NWN / 4, NWM * NWN / 4)))
void gemm_v3_f16_kernel(V2Params p) {
  constexpr int BN = 128, NT = 64 * NWM * NWN;
  constexpr int WTM = BM / NWM, WTN = BN / NWN, FM = WTM / 32, FN = WTN / 32;
  constexpr int A_DMA = BM / (8 * NWM * NWN);  // 1 KB DMA instructions per wave per tile
  constexpr int BCG = BN / 8, BROWS = NT / BCG, RPT = 64 / BROWS;  // 16 column groups; 4 or 2 rows
  static_assert(FM >= 2 && FN >= 1 && A_DMA >= 1 && (RPT == 4 || RPT == 2), "tile shape");
  constexpr bool has_gs = GS;

  __shared__ __align__(16) char sA0[BM * 128];
  __shared__ __align__(16) char sA1[BM * 128];
  __shared__ __align__(16) char sA2[BM * 128];
  __shared__ __align__(16) char sB0[BN * 128];
  __shared__ __align__(16) char sB1[BN * 128];
  __shared__ __align__(16) char sB2[BN * 128];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm0 = (wave / NWN) * WTM, wn0 = (wave % NWN) * WTN;
  int tm, tn;
  v2_tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = blockIdx.y * p.k_slice;
  const int ktiles = p.k_slice / 64;
  const int last = ktiles - 1;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  int a_off[A_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (wave * A_DMA + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_off[i] = (int)((int64_t)min(m0 + r, p.M - 1) * p.lda * 2) + c * 16;
  }
  auto issue_a = [&](int kt, char* sA) {
    const int soff = (k_begin + kt * 64) * 2;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) dma16(ra, sA + (wave * A_DMA + i) * 1024, a_off[i], soff);
  };

  const int brg = t % BROWS, bcg = t / BROWS;
  const int bn = min(n0 + bcg * 8, p.N - 8);
  __amdgpu_buffer_rsrc_t rb;
  int b_off;
  if (BMODE == kV2Int4) {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb * 4));
    b_off = (int)(((int64_t)brg * RPT * p.ldb + (bn >> 3)) * 4);
  } else {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb * 2));
    b_off = (int)(((int64_t)brg * RPT * p.ldb + bn) * 2);
  }
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(p.scales, has_gs ? (uint32_t)((int64_t)(p.K / p.group) * p.N * 2) : 16u);
  uint32_t breg[3][RPT][4];
  pk_u4v sreg[3] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  auto load_b = [&](int kt, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const int k0 = k_begin + kt * 64;
    if (BMODE == kV2Int4) {
      const int soff = (int)((int64_t)k0 * p.ldb * 4);
#pragma unroll
      for (int r = 0; r < RPT; ++r)
        breg[sl][r][0] = __builtin_amdgcn_raw_buffer_load_b32(rb, b_off + (int)(r * p.ldb * 4), soff, 0);
      if constexpr (has_gs) sreg[sl] = __builtin_amdgcn_raw_buffer_load_b128(rs, bn * 2, (k0 / p.group) * p.N * 2, 0);
    } else {
      const int soff = (int)((int64_t)k0 * p.ldb * 2);
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const pk_u4v v = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off + (int)(r * p.ldb * 2), soff, 0);
        breg[sl][r][0] = v[0]; breg[sl][r][1] = v[1]; breg[sl][r][2] = v[2]; breg[sl][r][3] = v[3];
      }
    }
  };
  // row r of tile kt's B words (int4), and the tile's scales with row 0
  auto load_b_row = [&](int kt, auto SLOT, int r) {
    constexpr int sl = decltype(SLOT)::value;
    const int k0 = k_begin + kt * 64;
    breg[sl][r][0] = __builtin_amdgcn_raw_buffer_load_b32(rb, b_off + (int)(r * p.ldb * 4), (int)((int64_t)k0 * p.ldb * 4), 0);
    if constexpr (has_gs) {
      if (r == 0) sreg[sl] = __builtin_amdgcn_raw_buffer_load_b128(rs, bn * 2, (k0 / p.group) * p.N * 2, 0);
    }
  };
  auto store_b = [&](auto SLOT, char* sB) {
    constexpr int sl = decltype(SLOT)::value;
    uint32_t col[8][RPT / 2];
    if (BMODE == kV2Int4) {
      uint32_t w[RPT];
#pragma unroll
      for (int r = 0; r < RPT; ++r) w[r] = breg[sl][r][0] ^ 0x88888888u;
      const pk_half2 bias = {(pk_half)1032.0f, (pk_half)1032.0f};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
#pragma unroll
        for (int r2 = 0; r2 < RPT / 2; ++r2) {
          const uint32_t pr = __builtin_amdgcn_perm(w[2 * r2 + 1], w[2 * r2], sel);
#pragma unroll
          for (int hs = 0; hs < 2; ++hs) {
            const int cidx = 2 * b + hs;
            const uint32_t nib = hs ? (pr >> 4) : pr;
            pk_half2 q = h2v((nib & 0x000f000fu) | 0x64006400u) - bias;  // exact codes
            if constexpr (has_gs) {
              const uint32_t sv = sreg[sl][cidx >> 1];
              const uint32_t s1 = (cidx & 1) ? (sv >> 16) : (sv & 0xffffu);
              q = q * h2v(s1 | (s1 << 16));
            }
            col[cidx][r2] = u32v(q);
          }
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int r2 = 0; r2 < RPT / 2; ++r2)
          col[c][r2] = __builtin_amdgcn_perm(breg[sl][2 * r2 + 1][c >> 1], breg[sl][2 * r2][c >> 1], sel);
      }
    }
    const int kb = RPT * brg * 2;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int n = bcg * 8 + c;
      if constexpr (RPT == 4) {
        pk_u2v v = {col[c][0], col[c][1]};
        *reinterpret_cast<pk_u2v*>(sB + swz(n, kb >> 4) + (kb & 15)) = v;
      } else {
        *reinterpret_cast<uint32_t*>(sB + swz(n, kb >> 4) + (kb & 15)) = col[c][0];
      }
    }
  };

  int aoff[FM][4], boff[FN][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i) aoff[i][ks] = swz(wm0 + 32 * i + (lane & 31), 2 * ks + (lane >> 5));
#pragma unroll
    for (int j = 0; j < FN; ++j) boff[j][ks] = swz(wn0 + 32 * j + (lane & 31), 2 * ks + (lane >> 5));
  }
  pk_f16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f16v){};
  // int4 B: the dequantisation of tile t+1 is written out in four pieces (one byte position
  // = two columns each) and woven between the MFMAs of tile t in source order, fenced by
  // scheduling barriers: a wave issues in order, so its VALU work overlaps its own matrix-pipe
  // work only when it sits between MFMAs. Fragment reads run one k-step ahead of the MFMAs
  // that use them.
  auto issue_a_part = [&](int kt, char* sA, int part) {  // the tile's DMAs spread over 4 k-steps
    const int soff = (k_begin + kt * 64) * 2;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i)
      if (i * 4 / A_DMA == part) dma16(ra, sA + (wave * A_DMA + i) * 1024, a_off[i], soff);
  };
  auto compute_store = [&](const char* sA, const char* sB, auto SLOT, char* sBn, int kta, char* sAn,
                           auto LSLOT) {
    constexpr int sl = decltype(SLOT)::value;
    pk_half8 af[2][FM], bf[2][FN];
    auto read = [&](int ks, int bsel) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[bsel][i] = *reinterpret_cast<const pk_half8*>(sA + aoff[i][ks]);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[bsel][j] = *reinterpret_cast<const pk_half8*>(sB + boff[j][ks]);
    };
    auto mfma2 = [&](int ks, int i) {  // fragment row i, every fragment column
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (BMODE == kV2BF16KN)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(pk_bf16x8, bf[ks & 1][j]), __builtin_bit_cast(pk_bf16x8, af[ks & 1][i]),
              acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[ks & 1][j], af[ks & 1][i], acc[i][j], 0, 0, 0);
      }
    };
    if constexpr (BMODE == kV2Int4) {
      uint32_t w[RPT];
      const pk_half2 bias = {(pk_half)1032.0f, (pk_half)1032.0f};
      uint32_t col[2][RPT / 2];  // the two columns of the current piece
      const int kb = RPT * brg * 2;
      // piece b, row pair r2: columns 2b (low nibbles) and 2b+1 (high nibbles)
      auto dq = [&](int b, int r2) {
        const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
        const uint32_t pr = __builtin_amdgcn_perm(w[2 * r2 + 1], w[2 * r2], sel);
        pk_half2 lo = h2v((pr & 0x000f000fu) | 0x64006400u) - bias;  // exact codes
        pk_half2 hi = h2v(((pr >> 4) & 0x000f000fu) | 0x64006400u) - bias;
        if constexpr (has_gs) {
          const uint32_t sv = sreg[sl][b];
          lo = lo * h2v(__builtin_amdgcn_perm(sv, sv, 0x01000100u));  // (s_lo, s_lo)
          hi = hi * h2v(__builtin_amdgcn_perm(sv, sv, 0x03020302u));  // (s_hi, s_hi)
        }
        col[0][r2] = u32v(lo);
        col[1][r2] = u32v(hi);
      };
      auto put = [&](int b) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int n = bcg * 8 + 2 * b + h;
          if constexpr (RPT == 4) {
            pk_u2v v = {col[h][0], col[h][1]};
            *reinterpret_cast<pk_u2v*>(sBn + swz(n, kb >> 4) + (kb & 15)) = v;
          } else {
            *reinterpret_cast<uint32_t*>(sBn + swz(n, kb >> 4) + (kb & 15)) = col[h][0];
          }
        }
      };
      read(0, 0);
#pragma unroll
      for (int r = 0; r < RPT; ++r) w[r] = breg[sl][r][0] ^ 0x88888888u;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks < 3) read(ks + 1, (ks + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        mfma2(ks, 0);
        __builtin_amdgcn_sched_barrier(0);
        issue_a_part(kta, sAn, ks);  // the next-but-one tile's A and B, spread over the k-steps
        if (ks < RPT) load_b_row(kta, LSLOT, ks);
        __builtin_amdgcn_sched_barrier(0);
        dq(ks, 0);
        __builtin_amdgcn_sched_barrier(0);
        mfma2(ks, 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RPT == 4) dq(ks, 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (FM == 4) {
          mfma2(ks, 2);
          __builtin_amdgcn_sched_barrier(0);
          put(ks);
          __builtin_amdgcn_sched_barrier(0);
          mfma2(ks, 3);
        } else {
          put(ks);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      read(0, 0);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks < 3) read(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < FM; ++i) mfma2(ks, i);
        __builtin_amdgcn_sched_barrier(0);
        issue_a_part(kta, sAn, ks);
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_sched_barrier(0);
      store_b(SLOT, sBn);
    }
  };

  // Per step this wave issues 5 (int4: 4 words + scales) or 4 (fp16) B loads, then 8 DMAs.
  // s_waitcnt vmcnt(V) expcnt(7) lgkmcnt(0): everything but the previous step's loads done.
  constexpr int kStepLoads = (BMODE == kV2Int4 ? RPT + (has_gs ? 1 : 0) : RPT) + A_DMA;
  constexpr int kWaitTile = (kStepLoads & 15) | (7 << 4) | ((kStepLoads >> 4) << 14);
  // prologue: tiles 0 and 1 in flight, tile 0's B in its stage
  load_b(0, pk_int_c<0>{});
  issue_a(0, sA0);
  load_b(min(1, last), pk_int_c<1>{});
  issue_a(min(1, last), sA1);
  store_b(pk_int_c<0>{}, sB0);
  auto step = [&](int kt, auto S, char* sAc, char* sBc, char* sAn, char* sBn1) {
    constexpr int st = decltype(S)::value;
    __builtin_amdgcn_s_waitcnt(kWaitTile);
    asm volatile("s_barrier" ::: "memory");
    if constexpr (BMODE != kV2Int4) load_b(min(kt + 2, last), pk_int_c<(st + 2) % 3>{});
    __builtin_amdgcn_sched_barrier(0);
    compute_store(sAc, sBc, pk_int_c<(st + 1) % 3>{}, sBn1, min(kt + 2, last), sAn,
                  pk_int_c<(st + 2) % 3>{});
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + 2 < ktiles; kt += 3) {
    step(kt, pk_int_c<0>{}, sA0, sB0, sA2, sB1);
    step(kt + 1, pk_int_c<1>{}, sA1, sB1, sA0, sB2);
    step(kt + 2, pk_int_c<2>{}, sA2, sB2, sA1, sB0);
  }
  if (kt < ktiles) step(kt, pk_int_c<0>{}, sA0, sB0, sA2, sB1);
  if (kt + 1 < ktiles) step(kt + 1, pk_int_c<1>{}, sA1, sB1, sA0, sB2);
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA into LDS outlives the waves
  mfma_drain();

  float* part = p.split > 1 ? p.partials + (int64_t)blockIdx.y * p.M * p.N : nullptr;
  const int esz = part ? 4 : (p.c_dtype == PK_F32 ? 4 : 2);
  const int em = lane & 31, en = 4 * (lane >> 5);
  // Through LDS when rows are 16-byte aligned: each wave stages its WTM x WTN block in a free
  // stage array (rows of WTN values, 16-byte chunks XOR-swizzled by row), then writes it back
  // row-contiguous, 16 bytes per lane, so a store instruction covers whole lines instead of
  // 8 or 16 bytes in each of 32 rows (measured on MI355X: the prefill GEMM 5-6% faster).
  char* const out_base = part ? reinterpret_cast<char*>(part) : reinterpret_cast<char*>(p.c);
  const int64_t ld_out = part ? p.N : p.ldc;
  if ((ld_out * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(out_base) & 15) == 0) {
    constexpr int STG = WTM * WTN * 4;  // bytes a wave stages (fp32 at most)
    static_assert(2 * STG <= BM * 128 && (2 * STG <= BN * 128 || STG <= BN * 128), "staging");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS reads are done
    __syncthreads();                     // and every other wave's: the stages are free
    char* sW;
    if (wave < 6) {
      char* const a2 = wave < 2 ? sA0 : wave < 4 ? sA1 : sA2;
      sW = a2 + (wave & 1) * STG;
    } else if constexpr (2 * STG <= BN * 128) {
      sW = sB0 + (wave - 6) * STG;
    } else {
      sW = wave == 6 ? sB0 : sB1;
    }
    with_dtype(part ? PK_F32 : p.c_dtype, [&](auto DT) {
      constexpr int dt = decltype(DT)::value;
      constexpr int E = dt == PK_F32 ? 4 : 2;
      constexpr int RB = WTN * E, NCH = RB / 16;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = 32 * i + em, col = 32 * j + 8 * q + en;
            const int byte = col * E;
            char* dst = sW + r * RB + ((((byte >> 4) ^ (r % NCH)) << 4) | (byte & 15));
            pk_f4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            if (!part) v = p.epi(v, n0 + wn0 + col);
            if constexpr (dt == PK_F32) {
              *reinterpret_cast<pk_f4*>(dst) = v;
            } else if constexpr (dt == PK_F16) {
              const pk_half4 hv = {(pk_half)v[0], (pk_half)v[1], (pk_half)v[2], (pk_half)v[3]};
              *reinterpret_cast<pk_u2v*>(dst) = __builtin_bit_cast(pk_u2v, hv);
            } else {
              const pk_u2v bv = {(uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
                                 (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16)};
              *reinterpret_cast<pk_u2v*>(dst) = bv;
            }
          }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // the wave's staging writes are in LDS
#pragma unroll
      for (int c0 = 0; c0 < WTM * NCH; c0 += 64) {
        const int idx = c0 + lane, r = idx / NCH, ch = idx % NCH;
        const pk_u4v val = *reinterpret_cast<const pk_u4v*>(sW + r * RB + ((ch ^ (r % NCH)) << 4));
        const int gm = m0 + wm0 + r, gn = n0 + wn0 + ch * (16 / E);
        if (gm < p.M && gn < p.N)  // N % 8 == 0: a chunk is all in or all out
          *PK_GLOBAL(pk_u4v, out_base + ((int64_t)gm * ld_out + gn) * E) = val;
      }
    });
    return;
  }
  const bool vec = part ? true
                        : (p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & (4 * esz - 1)) == 0);
  with_dtype(part ? PK_F32 : p.c_dtype, [&](auto DT) {
    constexpr int dt = decltype(DT)::value;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gm = m0 + wm0 + 32 * i + em;
          const int gn = n0 + wn0 + 32 * j + 8 * q + en;
          if (gm < p.M && gn < p.N) {
            pk_f4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            if (part) {
              store4_as<PK_F32>(part, (int64_t)gm * p.N + gn, v, true);
            } else {
              v = p.epi(v, gn);
              store4_as<dt>(p.c, (int64_t)gm * p.ldc + gn, v, vec);
            }
          }
        }
  });
}

// ---------------------------------------------------------------------------------------
// fp8 MFMA kernel (A e4m3 (M, K); B e4m3 (K, N) or (N, K)); BK = 128.
// ---------------------------------------------------------------------------------------
template <int BM, int BN, int WAVES_M, int WAVES_N, int BLAYOUT>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_v2_f8_kernel(V2Params p) {
  constexpr int NW = WAVES_M * WAVES_N, T = 64 * NW;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int A_DMA = BM / (8 * NW), B_DMA = BN / (8 * NW);
  constexpr int BCG = BN / 16;           // (K,N): 16-byte column groups
  constexpr int BROWS = T / BCG;         // row groups
  constexpr int RPT = 128 / BROWS;       // k rows per thread
  static_assert(RPT == 8 || RPT == 4, "(K,N) loader handles 8 or 4 rows per thread");

  __shared__ __align__(16) char sA0[BM * 128];
  __shared__ __align__(16) char sA1[BM * 128];
  __shared__ __align__(16) char sB0[BN * 128];
  __shared__ __align__(16) char sB1[BN * 128];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm0 = (wave / WAVES_N) * WTM, wn0 = (wave % WAVES_N) * WTN;
  int tm, tn;
  v2_tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int ktiles = p.K / 128;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda));
  int a_off[A_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (wave * A_DMA + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_off[i] = (int)((int64_t)min(m0 + r, p.M - 1) * p.lda) + c * 16;
  }
  auto issue_a = [&](int kt, char* sA) {
#pragma unroll
    for (int i = 0; i < A_DMA; ++i)
      dma16(ra, sA + (wave * A_DMA + i) * 1024, a_off[i], kt * 128);
  };

  // B (N, K): DMA like A. B (K, N): RPT rows x 16 bytes per thread through registers.
  __amdgpu_buffer_rsrc_t rb;
  int b_off[BLAYOUT == 1 ? B_DMA : 1];
  const int brg = t % BROWS, bcg = t / BROWS;
  const int bn = min(n0 + bcg * 16, p.N - 16);
  if (BLAYOUT == 1) {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.N * p.ldb));
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int r = (wave * B_DMA + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      b_off[i] = (int)((int64_t)min(n0 + r, p.N - 1) * p.ldb) + c * 16;
    }
  } else {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb));
    b_off[0] = (int)((int64_t)brg * RPT * p.ldb + bn);
  }
  pk_u4v breg[BLAYOUT == 0 ? RPT : 1];
  auto issue_b = [&](int kt, char* sB) {
    if (BLAYOUT == 1) {
#pragma unroll
      for (int i = 0; i < B_DMA; ++i)
        dma16(rb, sB + (wave * B_DMA + i) * 1024, b_off[i], kt * 128);
    } else {
      const int soff = (int)((int64_t)kt * 128 * p.ldb);
#pragma unroll
      for (int r = 0; r < RPT; ++r)
        breg[r] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[0] + (int)(r * p.ldb), soff, 0);
    }
  };
  // (K, N) B: RPT (8 or 4) rows x 16 bytes -> 16 columns x RPT k bytes, swizzled [n][k] LDS.
  auto tr4 = [](const uint32_t in[4], uint32_t out[4]) {  // 4x4 byte transpose
    const uint32_t t01a = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);
    const uint32_t t01b = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);
    const uint32_t t23a = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
    const uint32_t t23b = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(t23a, t01a, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(t23a, t01a, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(t23b, t01b, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(t23b, t01b, 0x07060302u);
  };
  auto store_b = [&](char* sB) {
    if constexpr (BLAYOUT == 0) {
      const int kb = RPT * brg;  // byte offset of the thread's k rows within the 128-byte row
#pragma unroll
      for (int d = 0; d < 4; ++d) {  // dword d = columns 4d..4d+3
        uint32_t lo[4], tl[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) lo[r] = breg[r][d];
        tr4(lo, tl);
        if constexpr (RPT == 8) {
          uint32_t hi[4], th[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) hi[r] = breg[4 + r][d];
          tr4(hi, th);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = bcg * 16 + 4 * d + q;
            pk_u2v v = {tl[q], th[q]};
            *reinterpret_cast<pk_u2v*>(sB + swz(n, kb >> 4) + (kb & 15)) = v;
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = bcg * 16 + 4 * d + q;
            *reinterpret_cast<uint32_t*>(sB + swz(n, kb >> 4) + (kb & 15)) = tl[q];
          }
        }
      }
    }
  };

  // operand offsets: per fragment, per k64 step, two 16-byte chunks (the lane's 32 bytes)
  int aoff[FM][2], boff[FN][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i) aoff[i][ks] = swz(wm0 + 32 * i + (lane & 31), 4 * ks + 2 * (lane >> 5));
#pragma unroll
    for (int j = 0; j < FN; ++j) boff[j][ks] = swz(wn0 + 32 * j + (lane & 31), 4 * ks + 2 * (lane >> 5));
  }
  // the second chunk (c + 1) of a row r sits at slot (c + 1) ^ s = (c ^ s) ^ 1 for even c
  auto chunk2 = [](int off) { return off ^ 16; };

  pk_f16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f16v){};

  auto compute = [&](const char* sA, const char* sB) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      pk_i8v bf[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const pk_u4v x0 = *reinterpret_cast<const pk_u4v*>(sB + boff[j][ks]);
        const pk_u4v x1 = *reinterpret_cast<const pk_u4v*>(sB + chunk2(boff[j][ks]));
        bf[j] = (pk_i8v){(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const pk_u4v x0 = *reinterpret_cast<const pk_u4v*>(sA + aoff[i][ks]);
        const pk_u4v x1 = *reinterpret_cast<const pk_u4v*>(sA + chunk2(aoff[i][ks]));
        const pk_i8v af = {(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af, acc[i][j], 0, 0, 0, 0, 0, 0);
      }
    }
  };

  issue_a(0, sA0);
  issue_b(0, sB0);
  store_b(sB0);
  __syncthreads();
  int kt = 0;
  // Scheduling barriers pin the next tile's loads at the top of each step (the compiler
  // otherwise issues them after the MFMAs, just before the barrier that waits for them).
  for (; kt + 1 < ktiles; kt += 2) {
    issue_b(kt + 1, sB1);
    issue_a(kt + 1, sA1);
    __builtin_amdgcn_sched_barrier(0);
    compute(sA0, sB0);
    __builtin_amdgcn_sched_barrier(0);
    store_b(sB1);
    __syncthreads();
    const int n2 = min(kt + 2, ktiles - 1);
    issue_b(n2, sB0);
    issue_a(n2, sA0);
    __builtin_amdgcn_sched_barrier(0);
    compute(sA1, sB1);
    __builtin_amdgcn_sched_barrier(0);
    store_b(sB0);
    __syncthreads();
  }
  if (kt < ktiles) compute(sA0, sB0);
  mfma_drain();

  // epilogue: fragments hold C^T (B is the first MFMA operand), so each register quad is
  // four consecutive columns of one row -> one 8- or 16-byte store
  const int esz = p.c_dtype == PK_F32 ? 4 : 2;
  const bool vec = p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & (4 * esz - 1)) == 0;
  const int em = lane & 31, en = 4 * (lane >> 5);
  with_dtype(p.c_dtype, [&](auto DT) {
    constexpr int dt = decltype(DT)::value;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gm = m0 + wm0 + 32 * i + em;
          const int gn = n0 + wn0 + 32 * j + 8 * q + en;  // N % 16 == 0: all four in or out
          if (gm < p.M && gn < p.N) {
            pk_f4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            v = p.epi(v, gn);
            store4_as<dt>(p.c, (int64_t)gm * p.ldc + gn, v, vec);
          }
        }
  });
}

// ---------------------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------------------
bool v2_f16_ok(int M, int N, int K, int k_slice, int group, bool has_gs, int64_t lda, int64_t ldb,
               bool int4) {
  if (M < 64 || N < 64 || N % 8 || k_slice % 64) return false;
  if (has_gs && group % 64) return false;
  // 32-bit buffer offsets
  if ((int64_t)M * lda * 2 >= (1ll << 31)) return false;
  if ((int64_t)K * ldb * (int4 ? 4 : 2) >= (1ll << 31)) return false;
  return true;
}

int v2_f16_launch(int bm, int bmode, const void* a, int64_t lda, const void* b, int64_t ldb,
                  const void* scales, int group, OutEpi epi, void* c, int c_dtype, int64_t ldc,
                  int M, int N, int K, int split, void* workspace, hipStream_t s,
                  bool partials_only) {
  V2Params p;
  p.a = a; p.lda = lda; p.b = b; p.ldb = ldb;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = group > 0 ? group : K;
  p.epi = epi; p.c = c; p.c_dtype = c_dtype; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K; p.split = split; p.k_slice = K / split;
  p.partials = split > 1 ? split_partials(workspace, partials_only) : nullptr;
  const int bn = 128;
  p.tiles_m = (int)cdiv(M, bm);
  p.tiles_n = (int)cdiv(N, bn);
  dim3 grid(p.tiles_m * p.tiles_n, split);
  const bool gs = scales != nullptr;
  // 8 waves, two per SIMD: 256-row tiles as 4 x 2 waves of 64 x 64 (measured 7% faster on
  // the 2048x4096x4096 prefill than 2 x 2 waves of 128 x 64), 128-row tiles as 2 x 4 waves of
  // 64 x 32 (measured 7-14% faster on the Llama-3-8B layers at M = 64 and 128 than 2 x 2
  // waves of 64 x 64).
  if (bmode == kV2Int4) {
    if (bm == 256) {
      if (gs) gemm_v3_f16_kernel<kV2Int4, true, 256, 4, 2><<<grid, 512, 0, s>>>(p);
      else gemm_v3_f16_kernel<kV2Int4, false, 256, 4, 2><<<grid, 512, 0, s>>>(p);
    } else {
      if (gs) gemm_v3_f16_kernel<kV2Int4, true, 128, 2, 4><<<grid, 512, 0, s>>>(p);
      else gemm_v3_f16_kernel<kV2Int4, false, 128, 2, 4><<<grid, 512, 0, s>>>(p);
    }
  } else if (bmode == kV2BF16KN) {
    if (bm == 256) gemm_v3_f16_kernel<kV2BF16KN, false, 256, 4, 2><<<grid, 512, 0, s>>>(p);
    else gemm_v3_f16_kernel<kV2BF16KN, false, 128, 2, 4><<<grid, 512, 0, s>>>(p);
  } else {
    if (bm == 256) gemm_v3_f16_kernel<kV2F16KN, false, 256, 4, 2><<<grid, 512, 0, s>>>(p);
    else gemm_v3_f16_kernel<kV2F16KN, false, 128, 2, 4><<<grid, 512, 0, s>>>(p);
  }
  PK_LAUNCH_CHECK("gemm v2 f16");
  if (split > 1 && !partials_only) return splitk_reduce(p.partials, split, M, N, epi, c, c_dtype, ldc, s);
  return PK_OK;
}

int v2_f8_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s) {
  V2Params p;
  p.a = a8; p.lda = lda; p.b = b8; p.ldb = ldb; p.scales = nullptr; p.group = K;
  p.epi = OutEpi(out_scale); p.c = c; p.c_dtype = c_dtype; p.ldc = ldc;
  p.M = M; p.N = N; p.K = K; p.split = 1; p.k_slice = K; p.partials = nullptr;
  const bool big = (int64_t)M * N >= (int64_t)2048 * 2048;
  const int bm = big ? 256 : 128, bn = big ? 256 : 128;
  p.tiles_m = (int)cdiv(M, bm);
  p.tiles_n = (int)cdiv(N, bn);
  const int grid = p.tiles_m * p.tiles_n;
  if (big) {
    if (b_layout == 1) gemm_v2_f8_kernel<256, 256, 2, 4, 1><<<grid, 512, 0, s>>>(p);
    else gemm_v2_f8_kernel<256, 256, 2, 4, 0><<<grid, 512, 0, s>>>(p);
  } else {
    if (b_layout == 1) gemm_v2_f8_kernel<128, 128, 2, 2, 1><<<grid, 256, 0, s>>>(p);
    else gemm_v2_f8_kernel<128, 128, 2, 2, 0><<<grid, 256, 0, s>>>(p);
  }
  PK_LAUNCH_CHECK("gemm v2 fp8");
  return PK_OK;
}

}  // namespace pk
