// W4A16 skinny GEMV (M <= 4) with deterministic split-K -- the HBM-bound decode path.
//
// Computes C[m, n] = tensor_scale * sum_k A[m, k] * q[k, n] * S[k / G, n] (+ bias[n]) for the packed
// layout of gemm_int4.pack_int4_n (gemm_int4.py:65-72) viewed as int32 words: word j of
// row k holds columns 8j..8j+7, nibble i = column 8j+i, two's complement.
//
// Work decomposition (one launch):
//   grid.x = column tiles of 256 columns (32 words = 128 contiguous bytes per row),
//   grid.y = split-K slices (contiguous K ranges of k_slice rows, as gemm_splitk.py:49-53).
//   A workgroup is 8 x RL lanes: 8 lanes span the 128-byte row segment with one 16-byte load
//   each (4 words = 32 columns per lane); RL row-lanes each own RPT consecutive rows per
//   step. Every lane keeps 32 column accumulators per activation row.
//
// Dequantisation without a conversion instruction per nibble:
//   * XOR each word with 0x88888888 turns the signed nibble v into u = v + 8 in [0, 15].
//   * A byte permute gathers the same byte of rows k and k+1 into the low bytes of the two
//     16-bit halves of one register; masking with 0x000F000F (or 0x00F000F0) leaves u in
//     the mantissa of two fp16 *subnormals*, i.e. the values u * 2^-24 (or u * 2^-20).
//   * v_dot2_f32_f16 multiplies that pair with the activation pair (x_k, x_k+1) and
//     accumulates in fp32: products are exact (11-bit x 4-bit significands) and fp16
//     subnormals are kept (the kernel's fp16 denormal mode is "preserve").
//   * Per step the column sum is rescaled by 2^24 (2^20), the +8 offset is removed with
//     -8 * sum(x) and the group scale is applied in fp32.
//
// Reduction: row-lanes inside a wave are folded with a reduce-scatter over lane masks
// 32/16/8, waves through LDS. With split-K each slice writes an fp32 partial row; the slices
// are then added in order 0..S-1 (bitwise reproducible, no floating-point atomics), either
// inside the same launch by the last slice of a column tile to arrive (the MFMA kernel below,
// when all slices of a tile share one XCD: gemv_finish_l2) or by a second small kernel
// (splitk_reduce_kernel) for this VALU kernel and the partials-only entry point.
#include "pk_internal.h"

namespace pk {

constexpr int kGemvCW = 8;          // lanes across a row segment
constexpr int kGemvTileWords = 32;  // words per column tile
constexpr int kGemvTileCols = 256;  // columns per column tile

struct GemvParams {
  const pk_half* a;
  int64_t lda;
  const uint32_t* qw;
  int64_t ldq;
  const pk_half* scales;  // (K/G, N) or null
  int group;
  OutEpi epi;  // tensor scale and optional bias
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int split, k_slice;
  int vec_ok;  // N % 32 == 0 and 16-byte aligned rows: whole-uint4 loads everywhere
  float* partials;  // (split, M, N) fp32 when split > 1; (split, M, npad) in the L2 handoff
  unsigned* counters;  // L2 handoff: arrival counter of tile t at counters[32 t]
  int tiles, npad;     // column tiles; tiles * 256
  QLayout ql;          // where the weight words live (the MFMA kernel; rows for the VALU one)
};

__device__ __forceinline__ pk_half2 as_half2(uint32_t v) { return __builtin_bit_cast(pk_half2, v); }

// Output stage shared by the GEMV kernels. `fold(m, col)` returns this workgroup's sum for
// activation row m and tile column col (after its __syncthreads). With split == 1 the value
// is scaled and stored, otherwise it goes to the (split, M, N) fp32 partials that
// splitk_reduce_kernel adds.
template <int MT, int NT, typename Fold>
__device__ __forceinline__ void gemv_finish(const GemvParams& p, int tile, int slice, int t,
                                            Fold fold) {
  const int col_base = tile * kGemvTileCols;
  for (int idx = t; idx < MT * kGemvTileCols; idx += NT) {
    const int m = idx / kGemvTileCols, col = idx % kGemvTileCols;
    if (m >= p.M || col_base + col >= p.N) continue;
    const float v = fold(m, col);
    if (p.split == 1)
      store_from_f32(p.c, p.c_dtype, (int64_t)m * p.ldc + col_base + col, p.epi(v, col_base + col));
    else
      p.partials[((int64_t)slice * p.M + m) * p.N + col_base + col] = v;
  }
}

// VEC: every lane owns 4 whole words with 16-byte aligned rows (N % 32 == 0), so weight
// loads need no per-lane branch. Loads are never predicated in the hot loop: a branch
// between a load and its first use makes the compiler wait for *all* outstanding loads at
// the join, which serialises memory and compute.
template <int MT, int RPT, int RL, bool HAS_GS, bool VEC>
__global__ __launch_bounds__(kGemvCW* RL) void w4a16_gemv_kernel(GemvParams p) {
  static_assert(RPT % 2 == 0 && RPT % 8 == 0, "RPT must be a multiple of 8");
  constexpr int NT = kGemvCW * RL;
  constexpr int NWAVES = (NT + 63) / 64;

  const int t = threadIdx.x;
  const int cl = t % kGemvCW, rl = t / kGemvCW;
  const int tile = blockIdx.x, slice = blockIdx.y;
  const int words_total = p.N >> 3;
  const int word0 = tile * kGemvTileWords + cl * 4;
  const int k_begin = slice * p.k_slice;
  const int k_end = min(k_begin + p.k_slice, p.K);
  constexpr bool has_gs = HAS_GS;

  float acc[MT][32];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[m][c] = 0.0f;

  for (int kb = k_begin + rl * RPT; kb < k_end; kb += RL * RPT) {
    // ---- issue all loads of this step: activations, weights in row order, then scales ----
    uint32_t xw[MT][RPT / 2];  // activation pairs (x_k, x_k+1) as packed fp16
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      // rows past M re-read row M-1; their results are never stored
      const uint4* xa = reinterpret_cast<const uint4*>(p.a + (int64_t)min(m, p.M - 1) * p.lda + kb);
#pragma unroll
      for (int v = 0; v < RPT / 8; ++v) {
        const uint4 q = xa[v];
        xw[m][4 * v + 0] = q.x; xw[m][4 * v + 1] = q.y;
        xw[m][4 * v + 2] = q.z; xw[m][4 * v + 3] = q.w;
      }
    }
    uint32_t w[RPT][4];
    if constexpr (VEC) {
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const pk_u4v v = __builtin_nontemporal_load(reinterpret_cast<const pk_u4v*>(p.qw + (int64_t)(kb + r) * p.ldq + word0));
        w[r][0] = v[0]; w[r][1] = v[1]; w[r][2] = v[2]; w[r][3] = v[3];
      }
    } else {
      const int wlast = words_total - 1;
#pragma unroll
      for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) w[r][j] = p.qw[(int64_t)(kb + r) * p.ldq + min(word0 + j, wlast)];
    }
    float sc[32];
    if constexpr (has_gs) {
      const int g = kb / p.group;
      const pk_half* srow = p.scales + (int64_t)g * p.N;
      if constexpr (VEC) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const pk_half8 h = __builtin_nontemporal_load(reinterpret_cast<const pk_half8*>(srow + (int64_t)word0 * 8 + 8 * v));
#pragma unroll
          for (int e = 0; e < 8; ++e) sc[8 * v + e] = (float)h[e];
        }
      } else {
#pragma unroll
        for (int c = 0; c < 32; ++c) sc[c] = (float)srow[min(word0 * 8 + c, p.N - 1)];
      }
    }

    // ---- dot products over the RPT rows ------------------------------------------------
    float part[MT][32];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < 32; ++c) part[m][c] = 0.0f;
#pragma unroll
    for (int r2 = 0; r2 < RPT / 2; ++r2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w0 = w[2 * r2][j] ^ 0x88888888u;
        const uint32_t w1 = w[2 * r2 + 1][j] ^ 0x88888888u;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          // bytes: [w0.byte_b, 0, w1.byte_b, 0]
          const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
          const uint32_t pr = __builtin_amdgcn_perm(w1, w0, sel);
          const pk_half2 lo = as_half2(pr & 0x000f000fu);  // column 8j+2b,   u * 2^-24
          const pk_half2 hi = as_half2(pr & 0x00f000f0u);  // column 8j+2b+1, u * 2^-20
          const int col = 8 * j + 2 * b;
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            const pk_half2 xv = as_half2(xw[m][r2]);
            part[m][col] = __builtin_amdgcn_fdot2(lo, xv, part[m][col], false);
            part[m][col + 1] = __builtin_amdgcn_fdot2(hi, xv, part[m][col + 1], false);
          }
        }
      }
    }
    // ---- undo the encoding and apply the group scale -----------------------------------
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float sx = 0.0f;
      const pk_half2 ones = {(pk_half)1.0f, (pk_half)1.0f};
#pragma unroll
      for (int r2 = 0; r2 < RPT / 2; ++r2) sx = __builtin_amdgcn_fdot2(as_half2(xw[m][r2]), ones, sx, false);
      const float off = -8.0f * sx;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const float v = __builtin_fmaf(part[m][c], (c & 1) ? 1048576.0f : 16777216.0f, off);
        if constexpr (has_gs) acc[m][c] = __builtin_fmaf(v, sc[c], acc[m][c]);
        else acc[m][c] += v;
      }
    }
  }

  // ---- fold row-lanes inside the wave: reduce-scatter over lane masks 32, 16, 8 ---------
  const int lane = t & 63;
  float red4[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float v16[16], v8[8];
    const bool u32 = (lane & 32) != 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float send = u32 ? acc[m][i] : acc[m][i + 16];
      const float keep = u32 ? acc[m][i + 16] : acc[m][i];
      v16[i] = keep + __shfl_xor(send, 32, 64);
    }
    const bool u16 = (lane & 16) != 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float send = u16 ? v16[i] : v16[i + 8];
      const float keep = u16 ? v16[i + 8] : v16[i];
      v8[i] = keep + __shfl_xor(send, 16, 64);
    }
    const bool u8 = (lane & 8) != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float send = u8 ? v8[i] : v8[i + 4];
      const float keep = u8 ? v8[i + 4] : v8[i];
      red4[m][i] = keep + __shfl_xor(send, 8, 64);
    }
  }
  // This lane now holds columns cbase..cbase+3 of its 32-column chunk.
  const int cbase = ((lane >> 5) & 1) * 16 + ((lane >> 4) & 1) * 8 + ((lane >> 3) & 1) * 4;

  // ---- fold waves through LDS ------------------------------------------------------------
  __shared__ float red[NWAVES][MT][kGemvTileCols];
  const int wave = t >> 6;
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][m][cl * 32 + cbase + i] = red4[m][i];
  __syncthreads();

  gemv_finish<MT, NT>(p, tile, slice, t, [&](int m, int col) {
    float v = red[0][m][col];
#pragma unroll
    for (int wv = 1; wv < NWAVES; ++wv) v += red[wv][m][col];
    return v;
  });
}

// ---------------------------------------------------------------------------------------
// MFMA variant (M <= 4, N % 32 == 0, K % 256 == 0, group % 64 == 0, aligned operands).
//
// Slices of 256 rows; a workgroup is 4 waves and each wave owns one 64-row x 128-byte block
// (lane: cl = lane % 8 picks 4 words = 32 columns, rl = lane / 8 picks 8 consecutive rows),
// so every wave issues all its loads at once and its rows lie in a single scale group.
// The products run on v_mfma_f32_16x16x32_f16, which also performs most of the row
// reduction:
//   * B operand of lane L: 8 fp16 values = the lane's 8 rows of one column pair. Output
//     column j = L % 16 of the MFMA sums lanes j, j+16, j+32, j+48, i.e. row lanes
//     rl = 2g + j/8 (g = 0..3) of column set cl = j % 8: four of the wave's eight row lanes.
//   * A operand of lane L: activation row m = L % 8 at the lane's own rows, so A-row
//     i = L % 16 carries the rows of parity i / 8, and C[m + 8p][j] is a complete sum over
//     the row lanes of parity p exactly when j / 8 == p. Lanes 0-7 (p = 0) and 40-47 (p = 1)
//     hold those outputs in their C registers m = 0..3; parities, waves and slices remain.
//   * B values are fp16 *subnormals* (MFMA keeps them exactly): after XOR 0x88888888 and a
//     byte permute of rows (k, k+1), a 16-bit half holds (u_lo + 16 u_hi) * 2^-24 for the
//     two nibbles of one byte (u = v + 8). With C_off = the MFMA of the constant 8 * 2^-24,
//       lo:  MFMA(A, halves & 0x000F000F, -C_off)    = 2^-24 * sum x * v_lo,
//       raw: MFMA(A, halves,              -17 C_off) and raw - lo = 2^-20 * sum x * v_hi,
//     so the nibble offset is folded into the accumulator input. Products are exact.
//   * The group scale multiplies each wave's column sums in the final fold (one scale per
//     wave and column), and the powers of two are applied there too.
// Per word that is 1 XOR, 2 permutes and 2 ANDs plus one MFMA, against 4 dot2 products, a
// 28-shuffle reduction and a per-step epilogue in the VALU kernel. Loads are raw buffer
// loads: a per-lane byte offset plus a wave-uniform row offset in a scalar register.
constexpr int kMfmaRows = 256;  // rows per workgroup = slice length
constexpr int kMfmaSeg = 36;    // LDS floats per 32-column segment (padding spreads banks)

// Occupancy hint: four workgroups per CU with one row block (three for the per-tensor
// variant of the one-launch form at M = 1, which would otherwise spill), else three.
template <int MT, bool HAS_GS, bool L2SPLIT, int RB>
__global__ __launch_bounds__(256, RB == 1 && (MT > 1 || HAS_GS || !L2SPLIT) ? 4 : 3)
void w4a16_gemv_mfma_kernel(GemvParams p) {
  constexpr int NW = 4;
  constexpr int WROWS = 64 * RB;  // rows per wave: RB blocks of 64, chained through the MFMAs
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int cl = lane & 7, rl = lane >> 3;
  int tile = blockIdx.x, slice = blockIdx.y;
  if constexpr (L2SPLIT) {
    xcd_tile_slice(p.split, tile, slice);
    if (tile >= p.tiles) return;
  }
  const int words_total = p.N >> 3;
  // the ragged last tile re-reads in-bounds words; those columns are never stored
  const int word0 = min(tile * kGemvTileWords + cl * 4, words_total - 4);
  const int kb = slice * (NW * WROWS) + wave * WROWS;  // this wave's rows: kb .. kb + WROWS - 1
  const int xrow = min(cl, p.M - 1);

  // Scales for the fold, requested first: thread t folds tile column t (a wave's rows lie in
  // one group).
  const int col_base = tile * kGemvTileCols;
  float sc[NW];
  if constexpr (HAS_GS) {
    const int scol = min(col_base + t, p.N - 1);
#pragma unroll
    for (int w = 0; w < NW; ++w)
      sc[w] = (float)__builtin_nontemporal_load(p.scales + (int64_t)((slice * NW * WROWS + w * WROWS) / p.group) * p.N + scol);
  }

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.qw, (uint32_t)((int64_t)p.K * p.ldq * 4));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  const int q_voff = rl * 8 * p.ql.row_bytes + (word0 >> 5) * p.ql.tile_bytes + (word0 & 31) * 4;
  pk_u4v xq[RB], w[RB][8];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    xq[rb] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(xrow * p.lda + rl * 8) * 2, (kb + 64 * rb) * 2, 0);
#pragma unroll
    for (int r = 0; r < 8; ++r)
      w[rb][r] = __builtin_amdgcn_raw_buffer_load_b128(rq, q_voff, qrow_off(p.ql, kb + 64 * rb + r), kPkLoadStream);
  }

  const pk_f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  const pk_u4v eight_u = {0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u};
  pk_half8 a[RB];
  pk_f4 coff = zero4;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    a[rb] = __builtin_bit_cast(pk_half8, xq[rb]);
    coff = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], __builtin_bit_cast(pk_half8, eight_u), coff, 0, 0, 0);
  }
  const pk_f4 cin_lo = -coff;
  const pk_f4 cin_raw = coff * -17.0f;
  // One row keeps all 16 byte columns of its sums in registers to the end; more rows leave
  // each j4's 4 byte columns in LDS as soon as they are complete, which keeps the live
  // registers (and so the waves per SIMD) at the one-row level.
  constexpr int JB = MT == 1 ? 16 : 4;
  __shared__ float red[NW][2][MT][8 * kMfmaSeg];
  const int par = lane >> 5;
  const bool valid = ((lane & 15) >> 3) == par && ((lane >> 4) & 1) == 0;  // lanes 0-7, 40-47
  float lo_out[MT][JB], hi_out[MT][JB];  // byte column jb = tile columns 2jb (lo), 2jb+1 (hi)
  // byte columns 2q, 2q+1 = tile columns 4q..4q+3 of the lane's 32-column chunk
  auto quad = [&](int r, int q) {
    const int j = MT == 1 ? 2 * q : 2 * (q & 1);
    return pk_f4{lo_out[r][j], hi_out[r][j], lo_out[r][j + 1], hi_out[r][j + 1]};
  };
#pragma unroll
  for (int j4 = 0; j4 < 4; ++j4) {
    uint32_t wx[RB][8];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 8; ++r) wx[rb][r] = w[rb][r][j4] ^ 0x88888888u;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
      pk_f4 clo = cin_lo, craw = cin_raw;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        pk_u4v raw, lo;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          raw[d] = __builtin_amdgcn_perm(wx[rb][2 * d + 1], wx[rb][2 * d], sel);
          lo[d] = raw[d] & 0x000f000fu;
        }
        clo = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], __builtin_bit_cast(pk_half8, lo), clo, 0, 0, 0);
        craw = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], __builtin_bit_cast(pk_half8, raw), craw, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < MT; ++r) {
        lo_out[r][MT == 1 ? 4 * j4 + b : b] = clo[r];
        hi_out[r][MT == 1 ? 4 * j4 + b : b] = craw[r] - clo[r];
      }
    }
    if constexpr (MT > 1) {
      if (valid) {
#pragma unroll
        for (int r = 0; r < MT; ++r)
#pragma unroll
          for (int q = 2 * j4; q < 2 * j4 + 2; ++q)
            *reinterpret_cast<pk_f4*>(&red[wave][par][r][cl * kMfmaSeg + 4 * q]) = quad(r, q);
      }
    }
  }

  // ---- fold parities and waves -------------------------------------------------------------
  if constexpr (MT == 1) {
    if (valid) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        *reinterpret_cast<pk_f4*>(&red[wave][par][0][cl * kMfmaSeg + 4 * q]) = quad(0, q);
    }
  }
  __syncthreads();
  auto fold = [&](int m, int col) {
    const int o = (col >> 5) * kMfmaSeg + (col & 31);
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) {
      const float part = red[wv][0][m][o] + red[wv][1][m][o];
      if constexpr (HAS_GS) v = __builtin_fmaf(part, sc[wv], v);
      else v += part;
    }
    return v * ((col & 1) ? 1048576.0f : 16777216.0f);  // exact: powers of two
  };
  if constexpr (L2SPLIT) gemv_finish_l2<MT>(p, tile, slice, t, fold);
  else gemv_finish<MT, 256>(p, tile, slice, t, fold);
}

// Output stage of the split-K GEMV whose slices hand off through one XCD's L2 (the grid
// layout and protocol of xcd_tile_slice / splitk_arrive): thread t owns tile column t.
template <int MT, typename Fold>
__device__ __forceinline__ void gemv_finish_l2(const GemvParams& p, int tile, int slice, int t,
                                               Fold fold) {
  const int col = tile * kGemvTileCols + t;
  float mine[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    mine[m] = m < p.M ? fold(m, t) : 0.0f;
    if (m < p.M) p.partials[((int64_t)slice * p.M + m) * p.npad + col] = mine[m];
  }
  if (!splitk_arrive(p.counters + 32 * tile, p.split)) return;
  if constexpr (MT == 1) {
    if (col >= p.N) return;
    const float v = splitk_sum(p.partials + col, (int64_t)p.M * p.npad, p.split, slice, mine[0]);
    store_from_f32(p.c, p.c_dtype, col, p.epi(v, col));
  } else {
    // Several rows: quads of 4 columns, all slices of a quad loaded at once (16 at a time),
    // so the last workgroup waits for ceil(MT / 4) rounds of loads, not MT.
    const int64_t plane = (int64_t)p.M * p.npad;
    for (int qi = t; qi < MT * (kGemvTileCols / 4); qi += 256) {
      const int m = qi / (kGemvTileCols / 4), c = tile * kGemvTileCols + (qi % (kGemvTileCols / 4)) * 4;
      if (m >= p.M || c >= p.N) continue;  // N % 32 == 0: whole quads
      const float* src = p.partials + (int64_t)m * p.npad + c;
      pk_f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int s0 = 0; s0 < p.split; s0 += 16) {
        pk_f4 pv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
          pv[u] = *reinterpret_cast<const pk_f4*>(src + (int64_t)min(s0 + u, p.split - 1) * plane);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (s0 + u == 0) v = pv[0];
          else if (s0 + u < p.split) v += pv[u];
        }
      }
      const int64_t o = (int64_t)m * p.ldc + c;
      v = p.epi(v, c);
#pragma unroll
      for (int e = 0; e < 4; ++e) store_from_f32(p.c, p.c_dtype, o + e, v[e]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Planning: which (RPT, RL, split) to run.
// ---------------------------------------------------------------------------------------
static bool gemv_config_ok(int K, int group, bool has_gs, int split, int rpt) {
  if (split < 1 || K % split) return false;
  const int ks = K / split;
  if (ks % rpt) return false;
  if (has_gs && (group % rpt)) return false;
  return true;
}

// Row blocks per wave the MFMA kernel uses for this slice length (0: not eligible). A wave's
// rows (64 per block) must lie in one quantisation group.
static int mfma_ok(int k_slice, int group, bool has_gs) {
  for (int rb = 1; rb <= 2; ++rb)
    if (k_slice == kMfmaRows * rb && (!has_gs || group % (64 * rb) == 0)) return rb;
  return 0;
}

// Automatic row blocks per wave: one (256-row slices) unless that makes more than 32 slices,
// then two (512-row slices). Measured at M = 1: 4096-deep layers are 1-12% faster with one
// block (16 slices), the 14336-deep down projection 7% faster with two (28 slices, not 56).
static int gemv_auto_rb(int K) { return K / kMfmaRows > 32 ? 2 : 1; }

static int pick_rl(int k_slice, int rpt) {
  const int steps = k_slice / rpt;  // row-lane steps available in one slice
  if (steps >= 32) return 32;
  if (steps >= 16) return 16;
  return 8;
}

bool gemv_plan(int M, int N, int K, int group, bool has_gs, int split_req, GemvPlan* out) {
  if (M < 1 || M > 4 || N % 8 || K % 16) return false;
  const int tiles = (int)cdiv(N, kGemvTileCols);
  const int rpt = 8;
  if (split_req > 0) {
    if (!gemv_config_ok(K, group, has_gs, split_req, rpt)) return false;
    const int ks = K / split_req;
    *out = {rpt, pick_rl(ks, rpt), split_req, ks, tiles, mfma_ok(ks, group, has_gs)};
    return true;
  }
  // Automatic: the MFMA kernel's 256-row slices when it applies; otherwise the smallest
  // split that puts >= 2048 waves in flight (8 per CU) with every row-lane busy, capped at
  // 32 slices.
  for (int rb = gemv_auto_rb(K); rb >= 1; --rb) {
    const int ks = kMfmaRows * rb;
    if (K % ks == 0 && mfma_ok(ks, group, has_gs) == rb) {
      *out = {rpt, pick_rl(ks, rpt), K / ks, ks, tiles, rb};
      return true;
    }
  }
  bool have = false;
  for (int s = 1; s <= 32; s *= 2) {
    if (!gemv_config_ok(K, group, has_gs, s, rpt)) continue;
    const int ks = K / s;
    const int rl = pick_rl(ks, rpt);
    *out = {rpt, rl, s, ks, tiles, mfma_ok(ks, group, has_gs)};
    have = true;
    const long waves = (long)tiles * s * (rl * kGemvCW / 64);
    if (waves >= 2048 && ks <= rl * rpt) break;
  }
  return have;
}

size_t gemv_workspace_bytes(const GemvPlan& pl, int M, int N) {
  if (pl.split <= 1) return 0;
  // room for the tile-padded partials of the L2 handoff, after the counters
  return kWsCounterBytes + (size_t)pl.split * M * pl.tiles * kGemvTileCols * sizeof(float);
}

template <int MT, int RPT, int RL>
static void launch_gemv_t(const GemvParams& p, int tiles, hipStream_t s) {
  dim3 grid(tiles, p.split);
  const bool gs = p.scales != nullptr;
  if (p.vec_ok) {
    if (gs) w4a16_gemv_kernel<MT, RPT, RL, true, true><<<grid, kGemvCW * RL, 0, s>>>(p);
    else w4a16_gemv_kernel<MT, RPT, RL, false, true><<<grid, kGemvCW * RL, 0, s>>>(p);
  } else {
    if (gs) w4a16_gemv_kernel<MT, RPT, RL, true, false><<<grid, kGemvCW * RL, 0, s>>>(p);
    else w4a16_gemv_kernel<MT, RPT, RL, false, false><<<grid, kGemvCW * RL, 0, s>>>(p);
  }
}

template <int MT>
static void launch_gemv_rl(const GemvParams& p, int rl, int tiles, hipStream_t s) {
  if (rl == 32) launch_gemv_t<MT, 8, 32>(p, tiles, s);
  else if (rl == 16) launch_gemv_t<MT, 8, 16>(p, tiles, s);
  else launch_gemv_t<MT, 8, 8>(p, tiles, s);
}

template <int MT, int RB>
static void launch_gemv_mfma_rb(const GemvParams& p, int tiles, hipStream_t s, bool l2split) {
  if (l2split) {
    const unsigned blocks = 8u * (unsigned)cdiv(tiles, 8) * (unsigned)p.split;
    if (p.scales) w4a16_gemv_mfma_kernel<MT, true, true, RB><<<blocks, 256, 0, s>>>(p);
    else w4a16_gemv_mfma_kernel<MT, false, true, RB><<<blocks, 256, 0, s>>>(p);
    return;
  }
  dim3 grid(tiles, p.split);
  if (p.scales) w4a16_gemv_mfma_kernel<MT, true, false, RB><<<grid, 256, 0, s>>>(p);
  else w4a16_gemv_mfma_kernel<MT, false, false, RB><<<grid, 256, 0, s>>>(p);
}

template <int MT>
static void launch_gemv_mfma(const GemvParams& p, int tiles, int rb, hipStream_t s, bool l2split) {
  if (rb == 2) launch_gemv_mfma_rb<MT, 2>(p, tiles, s, l2split);
  else launch_gemv_mfma_rb<MT, 1>(p, tiles, s, l2split);
}

// The MFMA kernel applies: 256- or 512-row slices within one group, 16-byte aligned operands
// with whole-uint4 rows, and buffers addressable with 32-bit offsets.
static bool gemv_mfma_ready(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                            int64_t ldq, const void* scales, int group, int M, int N, int K) {
  const int rb = pl.mfma;
  const bool vec = (reinterpret_cast<uintptr_t>(qw) & 15) == 0 && ldq % 4 == 0 && N % 32 == 0 &&
                   (scales == nullptr || (reinterpret_cast<uintptr_t>(scales) & 15) == 0);
  return rb >= 1 && pl.k_slice == kMfmaRows * rb && K % (kMfmaRows * rb) == 0 &&
         (scales == nullptr || group % (64 * rb) == 0) && vec &&
         (reinterpret_cast<uintptr_t>(a) & 15) == 0 && lda % 8 == 0 &&
         (int64_t)K * ldq * 4 < (1ll << 31) && (int64_t)M * lda * 2 < (1ll << 31);
}

bool gemv_tiled_ok(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                   int64_t ldq, const void* scales, int group, int M, int N, int K) {
  return N % kGemvTileCols == 0 && ldq == N / 8 &&
         gemv_mfma_ready(pl, a, lda, qw, ldq, scales, group, M, N, K);
}

int gemv_launch(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                int64_t ldq, const void* scales, int group, OutEpi epi, void* c,
                int c_dtype, int64_t ldc, int M, int N, int K, void* workspace,
                hipStream_t s, bool partials_only, bool tiled) {
  GemvParams p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.qw = qw;
  p.ldq = ldq;
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
  p.vec_ok = ((reinterpret_cast<uintptr_t>(qw) & 15) == 0 && ldq % 4 == 0 && N % 32 == 0 &&
              (scales == nullptr || (reinterpret_cast<uintptr_t>(scales) & 15) == 0)) ? 1 : 0;
  p.partials = pl.split > 1 ? split_partials(workspace, partials_only) : nullptr;
  p.counters = nullptr;
  p.tiles = pl.tiles;
  p.npad = pl.tiles * kGemvTileCols;
  p.ql = qlayout(tiled, ldq, N);
  const int rb = pl.mfma;
  const bool mfma = gemv_mfma_ready(pl, a, lda, qw, ldq, scales, group, M, N, K);
  if (tiled && !(mfma && N % kGemvTileCols == 0)) {
    set_error("w4a16 gemv: block-layout weights need the MFMA kernel (N %% 256 == 0, K %% 256 == 0)");
    return PK_EUNSUPPORTED;
  }
  if (mfma) {
    // Slices hand off through L2 unless the caller wants the partials themselves.
    const bool l2split = pl.split > 1 && !partials_only && pl.tiles <= kWsMaxTiles &&
                         splitk_in_l2_ok(s);
    if (l2split) p.counters = ws_counters(workspace);
    switch (M) {
      case 1: launch_gemv_mfma<1>(p, pl.tiles, rb, s, l2split); break;
      case 2: launch_gemv_mfma<2>(p, pl.tiles, rb, s, l2split); break;
      case 3: launch_gemv_mfma<3>(p, pl.tiles, rb, s, l2split); break;
      default: launch_gemv_mfma<4>(p, pl.tiles, rb, s, l2split); break;
    }
    PK_LAUNCH_CHECK("w4a16 gemv");
    if (l2split) return PK_OK;
  } else {
    switch (M) {
      case 1: launch_gemv_rl<1>(p, pl.rl, pl.tiles, s); break;
      case 2: launch_gemv_rl<2>(p, pl.rl, pl.tiles, s); break;
      case 3: launch_gemv_rl<3>(p, pl.rl, pl.tiles, s); break;
      default: launch_gemv_rl<4>(p, pl.rl, pl.tiles, s); break;
    }
  }
  PK_LAUNCH_CHECK("w4a16 gemv");
  if (pl.split > 1 && !partials_only)
    return splitk_reduce(p.partials, pl.split, M, N, epi, c, c_dtype, ldc, s);
  return PK_OK;
}

}  // namespace pk
