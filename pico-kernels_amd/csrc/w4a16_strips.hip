// W4A16 decode GEMV (1 <= M <= 8) on strip-layout weights: one workgroup per 16-column strip
// (or per two neighbouring strips, where the layer has strips enough) sums the whole of K
// itself, so a call is one launch with no split-K partials and no handoff between workgroups.
//
// Computes C[m, n] = tensor_scale * sum_k A[m, k] * q[k, n] * S[k / G, n] (+ bias[n]), the
// arithmetic of gemm_int4.int4_gemm_kernel (gemm_int4.py:21-55) with group scales.
//
// Strip layout (pk_w4a16_gemm_strips; a byte permutation of pack_int4_n's (K, N/2) bytes,
// gemm_int4.py:65-72, whose byte (k, c) holds columns 2c (low nibble) and 2c+1 (high)):
//   strip s = columns 16s .. 16s+15; its K rows are contiguous: 1 KB blocks b = rows
//   128b .. 128b+127 at byte (s * K/128 + b) * 1024. Inside a block, 16-byte chunk
//   L = 16g + 4rs + cps (g, rs, cps in 0..3) holds rows 32rs + 8g + e (e = 0..7) of the
//   column pairs 2cps (bytes 0..7, in row order e) and 2cps+1 (bytes 8..15), every nibble
//   stored as u = v + 8 (0..15, the two's-complement code v XOR 8).
//   Scales (group mode) are (N/16, K/G, 16) fp16: strip s's scales of group i at
//   (s * K/G + i) * 16.
// So lane L of a wave loads chunk L of a block: every wave load instruction reads 1 KB of
// contiguous weights, and a workgroup streams its strip's K/128 KB in one run.
//
// Products on v_mfma_f32_16x16x32_f16 (D = A x B, A 16x32, B 32x16): lane L supplies
// A[L % 16][8(L / 16) + e] and B[8(L / 16) + e][L % 16] and holds D[4(L / 16) + r][L % 16],
// r = 0..3. With lane L's chunk as its B operand (8 rows of one column pair), B column j
// = L % 16 carries column pair 2cps(j)+h of row set rs(j) = j / 4, and A row i carries
// activation row i % 4 at row set i / 4 (lane L loads the 8 activations of its own chunk's
// rows), so D[4rs + m][4rs + cps] is the sum over row set rs (32 rows) of activation row m
// times the column pair: it sits in register m of lane 20rs + cps. Rows 4..7 take a second
// MFMA set (activation rows i % 4 + 4).
//
// Dequantisation is exact, as in the split-K GEMV: a byte permute puts the byte of rows
// (e, e+1) in the low bytes of the two halves of a dword, i.e. fp16 subnormals
// (u_lo + 16 u_hi) * 2^-24 ("raw"), and masking with 0x000F000F leaves u_lo * 2^-24 ("lo").
// With O8 = the MFMA of the constant -8 * 2^-24 and O136 = 17 O8 as accumulator inputs,
//   lo  = MFMA(A, lo,  O8)   = 2^-24 * sum x * v_lo,
//   raw = MFMA(A, raw, O136), raw - lo = 2^-20 * sum x * v_hi
// (MFMA keeps fp16 subnormal inputs; products are exact). Each block's sums are scaled by
// their group scale in fp32 and added per lane in block order; the workgroup then adds its
// row sets and waves through LDS in a fixed order, so results are bitwise reproducible.
#include <new>

#include <hip/hip_ext.h>

#include "pk_internal.h"

namespace pk {

constexpr int kStripCols = 16;       // columns per strip
constexpr int kStripBlockRows = 128;  // rows per 1 KB block
constexpr int kStripMaxWaves = 16;
constexpr int kStripWaves8 = 8;  // waves per workgroup of the 5..8-row kernel

struct StripParams {
  const pk_half* a;
  int64_t lda;
  const uint8_t* qs;     // strip-layout codes
  const pk_half* ss;     // strip-layout scales, or null (per-tensor mode)
  int group;             // G (multiple of 32) with scales
  int group_shift;       // log2(G) when G is a power of two, else -1
  OutEpi epi;
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int kb;     // K / 128 blocks per strip
  int nw;     // waves per workgroup
  int iters;  // rounds of U blocks per wave
  int spx;    // units (strips, or pairs of strips) per XCD: ceil(units / 8)
};

// Group index of the 32-row row set at row `r0` (r0 % 32 == 0).
__device__ __forceinline__ int strip_group(const StripParams& p, int r0) {
  return p.group_shift >= 0 ? (r0 >> p.group_shift) : r0 / p.group;
}

#define PK_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// LDS staging (ALDS) is per wave: a wave's U blocks of activations (U x 128 columns of each
// of the M rows, as M runs of 256 U bytes) in a region of its own, so no wave waits for
// another. (Group scales are not staged: each lane loads its own 8 bytes per block beside its
// weights. Staged through LDS with the activations -- one 1 KB DMA per wave, of which a wave
// at group 128 uses 128 bytes -- the call ran 3-11% slower on MI355X: 4096 x 11008 M = 1
// 6.37 against 6.14 us, M = 4 8.40 against 7.46; o_proj 4096 x 4096 4.10 against 3.85.)
__host__ __device__ __forceinline__ int strip_wave_lds(int M, int U) { return (int)cdiv((int64_t)M * U * 256, 1024) * 1024; }
// A wave's partial sums for the end fold: 4 row sets x MT rows x 16 columns of fp32. With
// ALDS they overwrite the wave's own activation region (at least M * 256 bytes, rounded up to
// 1 KB, which holds the MT * 256 bytes whenever M > MT / 2); otherwise each wave has a
// region of this size.
__host__ __device__ __forceinline__ int strip_fold_lds(int MT) { return 4 * MT * 64; }
// A wave's LDS region: its staged activations (ALDS), later overwritten by its partials of
// each of its NS strips.
__host__ __device__ __forceinline__ int strip_wave_stride(int M, int MT, int U, bool alds, int ns) {
  const int fold = ns * strip_fold_lds(MT);
  return alds && strip_wave_lds(M, U) > fold ? strip_wave_lds(M, U) : fold;
}

// 16 bytes per lane, global -> LDS: lane L writes lds + 16 L.
__device__ __forceinline__ void strip_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS_PTR(lds), 16, voff, 0, 0, 0);
}

// MT: activation rows the kernel carries (1, 2, 4 or 8); U: 1 KB blocks per wave per round.
// ALDS: each wave DMAs its round's activations into its own LDS region ahead of its weight
// loads and reads them from there (M * U <= 32); otherwise every lane loads its own from
// global memory. Scales: every lane loads its own, beside its weights. NS: strips per
// workgroup. With NS = 2 each wave takes the same blocks of two neighbouring strips and
// multiplies both by one load (or one staged copy) of their activations, which halves the
// activation bytes the wave reads per weight byte. Up to 16 waves per workgroup with one strip
// (the 8-row kernel then runs U = 2 only, which keeps it within the 128 registers that
// allows), up to 8 with two.
template <int MT, int U, bool HAS_GS, bool ALDS, int NS = 1>
__global__ __launch_bounds__(64 * (NS == 1 ? kStripMaxWaves : kStripWaves8)) void w4a16_strip_kernel(StripParams p) {
  static_assert(NS == 1 || NS == 2, "one or two strips per workgroup");
  constexpr int MS = MT > 4 ? 2 : 1;            // MFMA sets of four activation rows
  constexpr int RR = MT < 4 ? MT : 4;           // registers of a set that carry rows
  extern __shared__ __align__(16) char strip_lds[];  // one region per wave
  // Workgroup b runs on XCD b % 8 (round-robin dispatch): XCD x takes the contiguous units
  // (strips, or pairs of strips) [x * spx, (x + 1) * spx), so each 128-byte line of the output
  // is written from one L2, except where two XCDs' ranges meet.
  const int nstrips = p.N / kStripCols;
  const int s0 = NS * ((int)(blockIdx.x & 7) * p.spx + (int)(blockIdx.x >> 3));
  if (s0 >= nstrips) return;
  // An odd strip count leaves the last pair one strip: it loads that strip twice and stores it once.
  const int ns_live = s0 + 1 < nstrips ? NS : 1;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4, cps = j & 3, rs = j >> 2;
  const int rowoff = 32 * rs + 8 * g;           // this lane's 8 rows inside a block

  const int64_t strip_bytes = (int64_t)p.kb * 1024;
  const int ngroups = HAS_GS ? p.K / p.group : 1;
  __amdgpu_buffer_rsrc_t rq[NS], rsc[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int s = s0 + (st < ns_live ? st : 0);
    rq[st] = make_rsrc(p.qs + (int64_t)s * strip_bytes, (uint32_t)strip_bytes);
    rsc[st] = make_rsrc(HAS_GS ? (const void*)(p.ss + (int64_t)s * ngroups * kStripCols) : (const void*)p.qs,
                        HAS_GS ? (uint32_t)(ngroups * kStripCols * 2) : 16u);
  }
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  const int wstride = strip_wave_stride(p.M, MT, U, ALDS, NS);
  char* const w_act = strip_lds + wave * wstride;
  int xoff[MS];  // this lane's activations inside block i: bytes of A (+ block), or of w_act
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
    const int m = min((lane & 3) + 4 * ms, p.M - 1);
    xoff[ms] = ALDS ? (m * U * 128 + rowoff) * 2 : (m * (int)p.lda + rowoff) * 2;
  }
  const pk_f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  const pk_u4v neg8 = {0x80088008u, 0x80088008u, 0x80088008u, 0x80088008u};      // -8 * 2^-24
  pk_f4 acc_lo[NS][MS][2], acc_hi[NS][MS][2];  // [strip][set][column pair h]: 2^-24 / 2^-20 units
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc_lo[st][ms][h] = acc_hi[st][ms][h] = zero4;

  for (int it = 0; it < p.iters; ++it) {
    const int b0 = (it * p.nw + wave) * U;
    if constexpr (ALDS) {
      // This round's activations (M runs of U * 128 columns from column b0 * 128, the blocks
      // past the strip clamped to its last), ahead of the weights.
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the previous round's LDS reads are done
      const int kp = U * 16, pieces = p.M * kp;  // 16-byte pieces
      for (int p0 = 0; p0 < pieces; p0 += 64) {
        const int pc = min(p0 + lane, pieces - 1), m = pc / kp;
        const int col = min(b0 * 128 + (pc % kp) * 8, p.K - 8);
        strip_dma16(ra, w_act + p0 * 16, (m * (int)p.lda + col) * 2);
      }
      asm volatile("" ::: "memory");
    }
    // ---- all loads of this round: U blocks of weights (and activations, scales) ----------
    pk_u4v w[NS][U], x[U][MS];
    pk_u2v sc[NS][U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int b = min(b0 + i, p.kb - 1);  // past the strip: re-read, contributes zero
#pragma unroll
      for (int st = 0; st < NS; ++st)
        w[st][i] = __builtin_amdgcn_raw_buffer_load_b128(rq[st], lane * 16, b * 1024, kPkLoadStream);
      if constexpr (!ALDS) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
          x[i][ms] = __builtin_amdgcn_raw_buffer_load_b128(ra, xoff[ms], b * (kStripBlockRows * 2), 0);
      }
      // The row set's group (per lane where G < 128). Non-temporal like the weights: measured
      // on MI355X at 4096 x 11008, M = 1, 6.15 -> 5.94 us against ordinary loads (sc0, sc1 or
      // both beside nt read the same).
      if constexpr (HAS_GS) {
#pragma unroll
        for (int st = 0; st < NS; ++st)
          sc[st][i] = __builtin_amdgcn_raw_buffer_load_b64(
              rsc[st], cps * 8 + strip_group(p, b * kStripBlockRows + 32 * rs) * (kStripCols * 2), 0,
              kPkLoadStream);
      }
    }
    if constexpr (ALDS) {
      // the wave's DMAs landed; its NS * U weight (and NS * U scale) loads, issued after them,
      // may fly
      constexpr int nv = (HAS_GS ? 2 : 1) * U * NS;
      static_assert(nv < 64, "vmcnt holds at most 63");
      __builtin_amdgcn_s_waitcnt((nv & 15) | (7 << 4) | (15 << 8) | ((nv >> 4) << 14));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int b = min(b0 + i, p.kb - 1);
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
          x[i][ms] = *reinterpret_cast<const pk_u4v*>(w_act + xoff[ms] + (b - b0) * (kStripBlockRows * 2));
      }
    }
    // Every load of the round issues before the products: left to itself the scheduler sinks
    // later blocks' scale and activation loads below earlier blocks' products (to reuse their
    // registers), and each round then waits a memory latency in its middle (measured at 8 rows
    // on MI355X: 4096 x 11008 14.0 -> 11.0 us, 14336 x 4096 12.5 -> 11.7 us).
    if constexpr (!ALDS) __builtin_amdgcn_sched_barrier(0);
    // ---- products, in block order -------------------------------------------------------
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (b0 + i >= p.kb) break;  // wave-uniform: the blocks past the strip (last round only)
      pk_half8 av[MS];
      pk_f4 o8[MS], o136[MS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        av[ms] = __builtin_bit_cast(pk_half8, x[i][ms]);
        o8[ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[ms], __builtin_bit_cast(pk_half8, neg8), zero4, 0, 0, 0);
        o136[ms] = o8[ms];  // 17 O8 (only the registers that carry rows are used)
#pragma unroll
        for (int r = 0; r < RR; ++r) o136[ms][r] = 17.0f * o8[ms][r];
      }
#pragma unroll
      for (int st = 0; st < NS; ++st) {  // O8 and O136 depend on the activations only
        float s_lo[2], s_hi[2];
        if constexpr (HAS_GS) {
          const pk_half4 hs = __builtin_bit_cast(pk_half4, sc[st][i]);
          s_lo[0] = (float)hs[0]; s_hi[0] = (float)hs[1];
          s_lo[1] = (float)hs[2]; s_hi[1] = (float)hs[3];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t d0 = w[st][i][2 * h], d1 = w[st][i][2 * h + 1];  // nibbles u = v + 8
          pk_u4v raw, lo;
          raw[0] = __builtin_amdgcn_perm(d0, d0, 0x0c010c00u);  // rows e = 0, 1
          raw[1] = __builtin_amdgcn_perm(d0, d0, 0x0c030c02u);  // rows 2, 3
          raw[2] = __builtin_amdgcn_perm(d1, d1, 0x0c010c00u);  // rows 4, 5
          raw[3] = __builtin_amdgcn_perm(d1, d1, 0x0c030c02u);  // rows 6, 7
#pragma unroll
          for (int d = 0; d < 4; ++d) lo[d] = raw[d] & 0x000f000fu;
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) {
            const pk_f4 clo = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[ms], __builtin_bit_cast(pk_half8, lo), o8[ms], 0, 0, 0);
            const pk_f4 craw = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[ms], __builtin_bit_cast(pk_half8, raw), o136[ms], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RR; ++r) {
              const float hi = craw[r] - clo[r];
              if constexpr (HAS_GS) {
                acc_lo[st][ms][h][r] = __builtin_fmaf(clo[r], s_lo[h], acc_lo[st][ms][h][r]);
                acc_hi[st][ms][h][r] = __builtin_fmaf(hi, s_hi[h], acc_hi[st][ms][h][r]);
              } else {
                acc_lo[st][ms][h][r] += clo[r];
                acc_hi[st][ms][h][r] += hi;
              }
            }
          }
        }
      }
    }
  }
  // (No MFMA drain before the fold: every MFMA result above is consumed by VALU inside the
  // loop, and the fold reads only the fp32 accumulators those VALU ops wrote.)

  // ---- row sets and waves, through LDS, in a fixed order ----------------------------------
  // Lane 20rs + cps holds columns 4cps .. 4cps+3 of row set rs in registers m % 4. Each wave
  // writes its 4 row sets; then thread (m, part, col) adds the partials of waves
  // part, part + 4, ... (row sets 0..3 each), and the four parts are added by two shuffles:
  // ((part 0 + part 1) + (part 2 + part 3)), the same tree on every call.
  // red(w, st)[rs][m][cps]: wave w's partials of strip st, in its own region (after its last
  // LDS reads of staged activations: a wave's LDS accesses complete in order).
  auto red = [&](int w, int st, int set, int m, int q) {
    return reinterpret_cast<pk_f4*>(strip_lds + w * wstride + st * strip_fold_lds(MT)) + (set * MT + m) * (kStripCols / 4) + q;
  };
  if ((lane >> 4) == rs) {
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int r = 0; r < RR; ++r)
          if (4 * ms + r < MT)
            *red(wave, st, rs, 4 * ms + r, cps) = pk_f4{acc_lo[st][ms][0][r], acc_hi[st][ms][0][r],
                                                        acc_lo[st][ms][1][r], acc_hi[st][ms][1][r]};
  }
  __syncthreads();
  const int rows = p.M < MT ? p.M : MT;
  // wave-uniform: one (strip, activation row) per wave
  for (int sm = wave; sm < ns_live * rows; sm += p.nw) {
    const int st = sm / rows, m = sm - st * rows;
    const int part = lane >> 4, col = lane & 15;
    const int kmax = (p.nw + 3) >> 2;  // wave-uniform
    // Every read first (addresses clamped to the last wave's region), one wait, then the adds
    // in the fixed order: the fold is one LDS round trip however many waves there are.
    float q4[kStripMaxWaves / 4][4];
#pragma unroll
    for (int k = 0; k < kStripMaxWaves / 4; ++k) {
      const int wv = min(part + 4 * k, p.nw - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) q4[k][q] = (*red(wv, st, q, m, col >> 2))[col & 3];
    }
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < kStripMaxWaves / 4; ++k) {
      if (k < kmax) {
        const bool live = part + 4 * k < p.nw;
#pragma unroll
        for (int q = 0; q < 4; ++q) v += live ? q4[k][q] : 0.0f;
      }
    }
    // The four parts (16-lane rows) added by row swaps instead of LDS shuffles: after
    // permlane16_swap(v, v) both rows of a pair hold (row 2i, row 2i+1), so their sum is the
    // pair's; permlane32_swap does the same for the halves. The same tree as before:
    // ((part 0 + part 1) + (part 2 + part 3)).
    {
      const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      v = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
      const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      v = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
    }
    if (part == 0) {
      v *= (col & 1) ? 1048576.0f : 16777216.0f;  // exact: powers of two
      const int n = (s0 + st) * kStripCols + col;
      store_from_f32(p.c, p.c_dtype, (int64_t)m * p.ldc + n, p.epi(v, n));
    }
  }
}

// ---------------------------------------------------------------------------------------
// Plan: U blocks per wave per round, as many waves as cover the strip in one round (at most
// 16), more rounds beyond that.
// ---------------------------------------------------------------------------------------
static int g_strip_u = 0;  // 0: automatic; 2, 4 or 8 fixes U (pk_w4a16_strips_config)

bool strips_shape_ok(int M, int N, int K, int group, bool has_gs) {
  if (M < 1 || M > 8 || N % kStripCols || K % kStripBlockRows || K < kStripBlockRows) return false;
  if (has_gs && (group % 32 || K % group || (group < 128 && 128 % group))) return false;
  return true;
}

// Blocks per wave, measured on MI355X at M = 1 (graphs over 40 rotating weight copies;
// 4096 x 11008: 2 / 4 / 8 blocks 7.26 / 6.40 / 6.93 us; 4096 x 6144: 5.04 / 4.95 / 5.25;
// 4096 x 14336: 8.98 / 7.76 / 8.07; 4096 x 4096: 4.29 / 4.23 / 4.06; 14336 x 4096: 7.53 /
// 7.62 / 8.12): 4 (8 waves per workgroup at K = 4096), 8 where the strips leave at most one
// workgroup per CU, 2 for deep layers (K > 8192: 16 waves, several rounds). More than two
// rows take at most 4 (the 4-row kernel spills with 8); more than four rows take 2 (the 8-row
// kernel's activation and accumulator registers double), whatever the configuration says.
static int strips_pick_u(int M, int N, int kb) {
  if (M > 4) return 2;
  int u = kb > 64 ? 2 : (N / kStripCols <= 256 ? 8 : 4);
  if (g_strip_u) u = g_strip_u;
  if (M > 2 && u > 4) u = 4;
  while (u > 2 && kb / u < 4) u /= 2;
  return u;
}

// 5..8 rows: 8 waves per workgroup, each lane loading its own activations and scales (no LDS
// staging). Measured on MI355X at M = 8 against 4 and 16 waves and against staging (graphs over
// rotating weight copies; 4096 x 6144 / 4096 x 4096 / 4096 x 14336 / 14336 x 4096 / 4096 x
// 11008): 8.09 / 5.56 / 13.3 / 11.7 / 10.9 us; staged, 9.4 / 7.3 / 16.8 / 19.5 / 14.2.
// Strips per workgroup (NS) and blocks per wave for them: at eight rows a wave reads two bytes
// of activations per weight byte, which costs more than the weights (measured: the same
// kernel with its activation loads left out ran qkv 8.3 -> 5.8 us, gate_up 13.4 -> 10.2), so
// layers with strips enough for it give each wave the same blocks of two strips and one load
// of their activations: with U = 2 (one workgroup per CU: 166 registers) from 320 to 512
// strips, with U = 1 (two per CU) above 768; never below 32 blocks (K < 4096), where the
// rounds are few. Measured at M = 8 (one strip / two): 4096 x 5120 8.46 / 7.19 us, 4096 x
// 6144 8.24 / 7.22, 4096 x 8192 8.08 / 7.59, 8192 x 6144 13.35 / 10.82, 8192 x 8192 13.81 /
// 11.97; U = 1: 4096 x 14336 13.36 / 12.02, 5120 x 13824 18.47 / 14.06, 4096 x 28672 22.31 /
// 21.64; left at one strip: 256 strips (4096 x 4096 5.55 against 6.95 for pairs, 14336 x
// 4096 11.73 against 16.1: half the CUs would idle), 688 and 768 (4096 x 11008 10.95 /
// 11.05, 4096 x 12288 10.95 / 10.98), 2048 x 8192 (5.58 / 5.70). Two to four rows (staged
// activations, the same U, at most 8 waves) pair on layers of more than 768 strips and 32..64
// blocks: M = 2 / 3 / 4 on 8192 x 14336 15.9 / 17.4 / 18.0 -> 12.8 / 14.0 / 14.5 us, 4096 x
// 14336 8.3 / 8.8 / 9.2 -> 7.6 / 8.3 / 8.5, 5120 x 13824 10.9 / 11.8 / 12.2 -> 10.7 / 11.3 /
// 11.7, 4096 x 28672 13.5 / 14.7 / 15.1 -> 13.2 / 14.2 / 14.6; elsewhere pairs at 1..4 rows
// ran slower or equal (4096 x 11008 M = 1 / 4: 6.21 / 7.63 against 7.11 / 8.53, 4096 x 4096
// M = 4 4.70 against 5.48, 4096 x 6144 within 2%).
static void strips_pick_pair(int M, int nstrips, int kb, int* ns, int* u) {
  *ns = 1;
  if (M > 4) *u = 2;
  if (kb < 32) return;
  if (M > 4) {
    if (nstrips >= 320 && nstrips <= 512) *ns = 2;
    else if (nstrips > 768) *ns = 2, *u = 1;
  } else if (M >= 2 && nstrips > 768 && kb <= 64 && *u <= 4) {
    *ns = 2;  // blocks per wave as for one strip (the two-strip kernels take U <= 4)
  }
}

// Activations staged per wave in LDS: at most 8 KB per wave (M * U <= 32).
static bool strips_alds(int M, int U) { return (int64_t)M * U <= 32; }

// Everything about a launch that depends on the shape and weights only.
struct StripPlan {
  StripParams p;  // a, c, ldc and M are filled in per call
  int u;
  int ns;  // strips per workgroup
  bool alds;
  size_t lds;
  dim3 grid, block;
};

static void strips_plan(const uint8_t* qs, const void* ss, int group, OutEpi epi, int c_dtype,
                        int M, int N, int K, int64_t lda, StripPlan* pl) {
  StripParams& p = pl->p;
  p.a = nullptr;
  p.lda = lda;
  p.qs = qs;
  p.ss = reinterpret_cast<const pk_half*>(ss);
  p.group = ss ? group : K;
  p.group_shift = -1;
  if (ss && (group & (group - 1)) == 0) p.group_shift = __builtin_ctz((unsigned)group);
  p.epi = epi;
  p.c = nullptr;
  p.c_dtype = c_dtype;
  p.ldc = 0;
  p.M = M;
  p.N = N;
  p.K = K;
  p.kb = K / kStripBlockRows;
  int u = strips_pick_u(M, N, p.kb), ns = 1;
  strips_pick_pair(M, N / kStripCols, p.kb, &ns, &u);
  const int waves_one_round = (int)cdiv(p.kb, u);
  const int max_waves = M > 4 || ns == 2 ? kStripWaves8 : kStripMaxWaves;  // the kernel's bound
  p.nw = waves_one_round < max_waves ? waves_one_round : max_waves;
  p.iters = (int)cdiv(p.kb, (int64_t)u * p.nw);
  const int mt = M == 1 ? 1 : M == 2 ? 2 : M <= 4 ? 4 : 8;
  pl->u = u;
  pl->ns = ns;
  pl->alds = M <= 4 && strips_alds(M, u) && (size_t)p.nw * strip_wave_lds(M, u) <= (64u << 10);
  pl->lds = (size_t)p.nw * strip_wave_stride(M, mt, u, pl->alds, ns);
  p.spx = (int)cdiv(cdiv(N / kStripCols, ns), 8);
  pl->grid = dim3(8 * p.spx);
  pl->block = dim3(64 * p.nw);
}

// start / stop: events the dispatch itself records as the kernel starts and ends (for timing;
// both null for a plain launch).
static int strips_run(const StripPlan& pl, const void* a, void* c, int64_t ldc, hipStream_t stream,
                      hipEvent_t start = nullptr, hipEvent_t stop = nullptr) {
  StripParams p = pl.p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.c = c;
  p.ldc = ldc;
  const int M = p.M, u = pl.u;
  const bool gs = p.ss != nullptr;
  // the two-strip kernels exist for U <= 4 at 2..4 rows and U <= 2 at 5..8 (strips_pick_pair)
  PK_REQUIRE(pl.ns == 1 || (M >= 2 && u <= (M > 4 ? 2 : 4)),
             "w4a16 gemv (strip layout): no two-strip kernel for M=%d U=%d", M, u);
  auto go = [&](auto MTc, auto Uc, auto AL, auto NSc) {
    constexpr int mt = decltype(MTc)::value, uu = decltype(Uc)::value, ns = decltype(NSc)::value;
    constexpr bool al = decltype(AL)::value != 0;
    auto kernel = gs ? w4a16_strip_kernel<mt, uu, true, al, ns> : w4a16_strip_kernel<mt, uu, false, al, ns>;
    if (start || stop)
      hipExtLaunchKernelGGL(kernel, pl.grid, pl.block, (uint32_t)pl.lds, stream, start, stop, 0, p);
    else
      kernel<<<pl.grid, pl.block, pl.lds, stream>>>(p);
  };
  auto by_u = [&](auto MTc, auto AL) {
    constexpr int mt = decltype(MTc)::value;
    constexpr pk_int_c<1> one{};
    auto go1 = [&](auto MT2, auto U2, auto AL2) {
      if (pl.ns == 2) go(MT2, U2, AL2, pk_int_c<2>{});
      else go(MT2, U2, AL2, one);
    };
    if constexpr (mt == 8) {  // U = 2 with one strip per workgroup; U = 2 or 1 with two
      if (pl.ns == 1) go(MTc, pk_int_c<2>{}, AL, one);
      else if (u == 2) go(MTc, pk_int_c<2>{}, AL, pk_int_c<2>{});
      else go(MTc, pk_int_c<1>{}, AL, pk_int_c<2>{});
    } else if constexpr (mt == 4) {  // U <= 4 (strips_pick_u)
      if (u == 2) go1(MTc, pk_int_c<2>{}, AL);
      else go1(MTc, pk_int_c<4>{}, AL);
    } else if constexpr (mt == 2) {  // two strips: U <= 4 (kb <= 64, more than 256 strips)
      if (u == 2) go1(MTc, pk_int_c<2>{}, AL);
      else if (u == 4) go1(MTc, pk_int_c<4>{}, AL);
      else go(MTc, pk_int_c<8>{}, AL, one);
    } else {
      if (u == 2) go(MTc, pk_int_c<2>{}, AL, one);
      else if (u == 4) go(MTc, pk_int_c<4>{}, AL, one);
      else go(MTc, pk_int_c<8>{}, AL, one);
    }
  };
  auto by_m = [&](auto AL) {
    if (M == 1) by_u(pk_int_c<1>{}, AL);
    else if (M == 2) by_u(pk_int_c<2>{}, AL);
    else by_u(pk_int_c<4>{}, AL);
  };
  if (M > 4) by_u(pk_int_c<8>{}, pk_int_c<0>{});  // eight rows: never staged
  else if (pl.alds) by_m(pk_int_c<1>{});
  else by_m(pk_int_c<0>{});
  PK_LAUNCH_CHECK("w4a16 gemv (strip layout)");
  return PK_OK;
}

int strips_launch(const void* a, int64_t lda, const uint8_t* qs, const void* ss, int group,
                  OutEpi epi, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                  hipStream_t stream) {
  StripPlan pl;
  strips_plan(qs, ss, group, epi, c_dtype, M, N, K, lda, &pl);
  return strips_run(pl, a, c, ldc, stream);
}

bool strips_config_set(int u) {
  if (u != 0 && u != 2 && u != 4 && u != 8) return false;
  g_strip_u = u;
  return true;
}

}  // namespace pk

using namespace pk;

extern "C" int pk_w4a16_strips_config(int blocks_per_wave) {
  PK_REQUIRE(strips_config_set(blocks_per_wave),
             "pk_w4a16_strips_config: %d is not 0 (automatic), 2, 4 or 8", blocks_per_wave);
  return PK_OK;
}

extern "C" int pk_w4a16_strips_plan(int M, int N, int K, int* strips_per_workgroup,
                                    int* blocks_per_wave, int* waves) {
  PK_REQUIRE(M >= 1 && M <= 8, "pk_w4a16_strips_plan: M=%d (the strip layout serves 1..8 rows)", M);
  PK_REQUIRE(N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0,
             "pk_w4a16_strips_plan: needs N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)", N, K);
  StripPlan pl;
  strips_plan(nullptr, nullptr, K, OutEpi(1.0f, nullptr, PK_F32), PK_F32, M, N, K, K, &pl);
  if (strips_per_workgroup) *strips_per_workgroup = pl.ns;
  if (blocks_per_wave) *blocks_per_wave = pl.u;
  if (waves) *waves = pl.p.nw;
  return PK_OK;
}

namespace {
int check_strips(const char* name, const void* a, int64_t lda, const uint8_t* qstrips,
                 const void* sstrips, int group_size, const void* bias, int bias_dtype,
                 const void* c, int c_dtype, int64_t ldc, int M, int N, int K) {
  auto al = [](const void* q, unsigned b) { return (reinterpret_cast<uintptr_t>(q) & (b - 1)) == 0; };
  PK_REQUIRE(qstrips != nullptr, "%s: null weights", name);
  PK_REQUIRE(M >= 1 && M <= 8, "%s: M=%d (the strip layout serves 1..8 rows)", name, M);
  PK_REQUIRE(N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0,
             "%s: needs N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)", name, N, K);
  PK_REQUIRE(sstrips == nullptr || strips_shape_ok(M, N, K, group_size, true),
             "%s: group_size=%d must be a multiple of 32 dividing K=%d and either divide 128 or "
             "be a multiple of it", name, group_size, K);
  PK_REQUIRE(a == nullptr || (lda >= K && lda % 8 == 0 && al(a, 16)),
             "%s: A rows must be 16-byte aligned", name);
  PK_REQUIRE((int64_t)M * lda * 2 < (1ll << 31), "%s: A beyond 2 GiB", name);
  PK_REQUIRE((int64_t)K * 8 < (1ll << 31), "%s: K=%d too large", name, K);
  PK_REQUIRE(al(qstrips, 16) && (sstrips == nullptr || al(sstrips, 8)),
             "%s: weights must be 16-byte and scales 8-byte aligned", name);
  PK_REQUIRE(c == nullptr || ldc >= N, "%s: ldc < N", name);
  PK_REQUIRE(c_dtype == PK_F32 || c_dtype == PK_F16 || c_dtype == PK_BF16,
             "%s: output dtype %d", name, c_dtype);
  PK_REQUIRE(bias == nullptr || bias_dtype == PK_F32 || bias_dtype == PK_F16 || bias_dtype == PK_BF16,
             "%s: bias dtype %d", name, bias_dtype);
  return PK_OK;
}

// A prepared call: the plans of one set of weights for M = 1..8 at one lda (made once, read
// only afterwards, so concurrent runs on different streams may share it).
struct StripsPrepared {
  StripPlan plan[8];  // by M - 1
  int N;
  int64_t lda;
};
}  // namespace

extern "C" int pk_w4a16_gemm_strips(const void* a, int64_t lda, const uint8_t* qstrips,
                                    const void* sstrips, int group_size, float tensor_scale,
                                    const void* bias, int bias_dtype, void* c, int c_dtype,
                                    int64_t ldc, int M, int N, int K, void* stream) {
  PK_REQUIRE(a != nullptr && c != nullptr, "pk_w4a16_gemm_strips: null pointer");
  const int rc = check_strips("pk_w4a16_gemm_strips", a, lda, qstrips, sstrips, group_size, bias,
                              bias_dtype, c, c_dtype, ldc, M, N, K);
  if (rc != PK_OK) return rc;
  return strips_launch(a, lda, qstrips, sstrips, group_size, OutEpi(tensor_scale, bias, bias_dtype),
                       c, c_dtype, ldc, M, N, K, (hipStream_t)stream);
}

extern "C" void* pk_w4a16_strips_prepare(const uint8_t* qstrips, const void* sstrips,
                                         int group_size, float tensor_scale, const void* bias,
                                         int bias_dtype, int c_dtype, int N, int K, int64_t lda) {
  if (check_strips("pk_w4a16_strips_prepare", nullptr, lda, qstrips, sstrips, group_size, bias,
                   bias_dtype, nullptr, c_dtype, N, 1, N, K) != PK_OK)
    return nullptr;
  auto* h = new (std::nothrow) StripsPrepared();
  if (h == nullptr) {
    set_error("pk_w4a16_strips_prepare: out of host memory");
    return nullptr;
  }
  h->N = N;
  h->lda = lda;
  for (int m = 1; m <= 8; ++m)
    strips_plan(qstrips, sstrips, group_size, OutEpi(tensor_scale, bias, bias_dtype), c_dtype, m,
                N, K, lda, &h->plan[m - 1]);
  return h;
}

namespace {
int strips_run_checked(const char* name, void* prepared, const void* a, void* c, int64_t ldc,
                       int M, void* stream, void* start, void* stop) {
  auto* h = static_cast<StripsPrepared*>(prepared);
  PK_REQUIRE(h != nullptr && a != nullptr && c != nullptr, "%s: null pointer", name);
  PK_REQUIRE(M >= 1 && M <= 8, "%s: M=%d (the strip layout serves 1..8 rows)", name, M);
  PK_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15) == 0, "%s: A must be 16-byte aligned", name);
  PK_REQUIRE(ldc >= h->N, "%s: ldc < N", name);
  PK_REQUIRE((int64_t)M * h->lda * 2 < (1ll << 31), "%s: A beyond 2 GiB", name);
  return strips_run(h->plan[M - 1], a, c, ldc, (hipStream_t)stream, (hipEvent_t)start,
                    (hipEvent_t)stop);
}
}  // namespace

extern "C" int pk_w4a16_strips_run(void* prepared, const void* a, void* c, int64_t ldc, int M,
                                   void* stream) {
  return strips_run_checked("pk_w4a16_strips_run", prepared, a, c, ldc, M, stream, nullptr, nullptr);
}

extern "C" int pk_w4a16_strips_run_events(void* prepared, const void* a, void* c, int64_t ldc,
                                          int M, void* stream, void* start_event,
                                          void* stop_event) {
  return strips_run_checked("pk_w4a16_strips_run_events", prepared, a, c, ldc, M, stream,
                            start_event, stop_event);
}

extern "C" void pk_w4a16_strips_release(void* prepared) {
  delete static_cast<StripsPrepared*>(prepared);
}
