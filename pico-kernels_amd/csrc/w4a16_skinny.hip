// W4A16 matmul for 5 <= M <= 128 activation rows: the HBM-bound middle between the GEMV
// (M <= 4) and the LDS-tiled GEMM. C = tensor_scale * A (M, K) fp16 @ deq(W) (K, N) (+ bias), W in
// the packed layout of gemm_int4.pack_int4_n (gemm_int4.py:65-72) viewed as int32 words
// (word j of row k = columns 8j..8j+7, nibble i = column 8j+i) and the group scales of
// quantize.rtn_layer along K (quantize.py:63-68).
//
// Work decomposition: grid.x = column tiles (x row parts), grid.y = split-K slices of k_slice
// rows (contiguous, as gemm_splitk.py:49-53). The NW waves of a workgroup (4 or 8) take
// consecutive 1/NW parts of the slice; a wave walks its rows in k-steps of 32 with several
// k-steps of loads in flight (no LDS staging: weights go straight to registers). A workgroup
// covers MB 16-row activation blocks (1, 2 or 4); above 64 rows two row parts share each
// (tile, slice), their workgroups placed on one XCD so the second reads the weights from L2.
//
// Per k-step a lane (j = lane % 16, g = lane / 16) loads CPL / 2 bytes (CPL = 16 or 8
// columns: CPL*j .. CPL*j + CPL-1 of the tile) of the 8 rows 8g..8g+7, plus 16 bytes of
// activations per block (row j of the block, the same 8 k). That is exactly the operand layout
// of v_mfma_f32_16x16x32_f16: lane L supplies A[L%16][8g+d] and B[8g+d][L%16] for d = 0..7, so
// MFMA number c (c = 0..CPL-1) multiplies the activations by weight column CPL*j + c of lane j,
// and the 16 x 16 result lands in lane L as rows 4g..4g+3 of that column. No data crosses
// lanes. Tiles are 16 * CPL columns: 256 (one 128-byte line per row) or 128 (half the
// accumulators, so four blocks fit in registers).
//
// Dequantisation without a conversion per nibble (the arithmetic of the M <= 4 GEMV): XOR
// 0x88888888 turns each signed nibble v into u = v + 8; a byte permute gathers one byte of rows
// (2d, 2d+1) into the two 16-bit halves of a register, i.e. the fp16 subnormals
// (u_lo + 16 u_hi) * 2^-24, and masking with 0x000F000F leaves u_lo * 2^-24. The MFMA keeps
// fp16 subnormals and forms the products exactly, so per byte two MFMAs give
//   L = sum x * u_lo * 2^-24   and   R = sum x * (u_lo + 16 u_hi) * 2^-24,
// and with O = sum x * 8 * 2^-24 (one more MFMA per k-step against a constant operand)
//   sum x * v_lo = (L - O) * 2^24,   sum x * v_hi = (R - L - 16 O) * 2^20.
// A wave's rows lie in one quantisation group, so its fp32 result is scaled once per column
// at the end (exact powers of two folded into the scale); with two 16-row blocks and 8 columns
// per lane a wave may instead take several whole 128-row groups, scaling and adding each
// group's sums at its boundary (fewer slices on deep or wide layers).
//
// Reduction: the waves' tiles are added in LDS in a fixed order. With split-K and one 16-row
// block the slices of a column tile hand off through one XCD's L2 inside the launch, as the
// M <= 4 GEMV does: a 1-D grid places the split * row_parts workgroups of a tile on one XCD
// (xcd = workgroup id mod 8), each writes its fp32 partial block, waits for the stores and
// bumps the tile's arrival counter; the last to arrive adds the split partials in slice order
// 0..split-1 -- the arithmetic of splitk_reduce_kernel, so the result is bitwise that of the
// two-launch form -- and stores C. More rows, the partials-only entry point, and partitions
// whose XCD count does not divide 8 (or PK_SPLITK_IN_L2=0) write (split, M, N) partials
// that splitk_reduce_kernel adds in a second launch.
#include <atomic>
#include <cstdio>
#include <cstdlib>

#include "pk_internal.h"

namespace pk {

constexpr int kSkStep = 32;  // rows per k-step (4 lane groups x 8 rows)
constexpr int kSkPad = 4;    // LDS row padding (floats)

struct SkinnyParams {
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
  int tiles, row_parts;
  float* partials;  // (split, M, N) fp32 when split > 1; (split, M, npad) in the L2 handoff
  unsigned* counters;  // arrival counters of the L2 handoff, one 128-byte line per (tile, part)
  int npad;            // tiles * tile columns
  QLayout ql;          // where the weight words live
};

template <int MB, int WPL>
struct SkStep {
  uint32_t w[8][WPL];  // rows 8g..8g+7, the lane's WPL words of the tile
  pk_u4v x[MB];        // activations: row j of each 16-row block, k = 8g..8g+7
};

// MB: 16-row activation blocks per workgroup; CPL: columns per lane (16: 8-byte weight loads,
// 256-column tiles; 8: 4-byte loads, 128-column tiles, half the accumulators per block);
// NW: waves per workgroup, each taking 1/NW of the slice's rows. MG: the wave's rows span
// several 128-row groups; its sums are scaled and added up at every group boundary.
template <int MB, int CPL, int NW, bool HAS_GS, int PD, int OCC, bool L2, bool MG>
__global__ __launch_bounds__(64 * NW, OCC) void w4a16_skinny_kernel(SkinnyParams p) {
  constexpr int TC = 16 * CPL;  // tile columns
  constexpr int WPL = CPL / 8;  // words per lane and row
  constexpr int NB = NW / 2;    // LDS reduction buffers
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  // Workgroups 8 ids apart run on one XCD (round-robin dispatch; grid widths are multiples of
  // 8), x = b % 8 naming it. Row parts of one (tile,
  // slice) are dispatched next to each other on one XCD, so the second part's weight reads
  // hit that XCD's L2; so are the two 128-column tiles that share each 128-byte weight line
  // (8 columns per lane): one XCD reads the line from HBM once instead of two XCDs each
  // reading all of it. In the one-launch split-K form the 1-D grid also keeps every slice of a
  // tile on that XCD.
  int part, tile, slice;
  {
    const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int per = (L2 ? p.split : 1) * p.row_parts;  // units per tile on one XCD
    const int u = (CPL == 8 ? j >> 1 : j) % per;
    const int g = (CPL == 8 ? j >> 1 : j) / per;
    tile = CPL == 8 ? 16 * g + 2 * x + (j & 1) : 8 * g + x;
    part = u % p.row_parts;
    slice = L2 ? u / p.row_parts : (int)blockIdx.y;
  }
  if (tile >= p.tiles) return;
  const int m0 = part * MB * 16;
  const int words_total = p.N >> 3;
  // The ragged last tile re-reads in-bounds words; those columns are never stored.
  const int word0 = min(tile * (TC / 8) + WPL * j, words_total - WPL);
  const int rows_w = p.k_slice / NW;
  const int nsteps = rows_w / kSkStep;
  const int kb = slice * p.k_slice + wave * rows_w;

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.qw, (uint32_t)((int64_t)p.K * p.ldq * 4));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(HAS_GS ? (const void*)p.scales : (const void*)p.qw,
                HAS_GS ? (uint32_t)((int64_t)(p.K / p.group) * p.N * 2) : 0u);
  // a lane's words lie in one 256-column tile (word0 % 32 + WPL <= 32)
  const int q_voff = 8 * g * p.ql.row_bytes + (word0 >> 5) * p.ql.tile_bytes + (word0 & 31) * 4;
  int a_voff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    a_voff[mb] = (int)(min(m0 + mb * 16 + j, p.M - 1) * p.lda + 8 * g) * 2;
  // The wave's (first) group kb / group: its CPL column scales, requested first.
  pk_u4v sraw[WPL];
#pragma unroll
  for (int i = 0; i < WPL; ++i) sraw[i] = pk_u4v{0u, 0u, 0u, 0u};
  if constexpr (HAS_GS) {
    const int srow = (kb / p.group) * p.N * 2;
#pragma unroll
    for (int i = 0; i < WPL; ++i)
      sraw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, word0 * 16 + 16 * i, srow, kPkLoadStream);
  }

  // Weights and scales load non-temporally (read once per call; measured on MI355X on the
  // Llama-3-8B layers at M = 32 against ordinary loads: qkv 12.15 -> 11.54 us, o_proj 10.37 ->
  // 9.72, down 18.76 -> 17.83; o_proj at M = 128 16.76 -> 15.96). Activations stay cached:
  // every workgroup reads them.
  auto load = [&](SkStep<MB, WPL>& b, int s) {
    const int k0 = kb + s * kSkStep;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      if constexpr (WPL == 2) {
        const pk_u2v v = __builtin_amdgcn_raw_buffer_load_b64(rq, q_voff, qrow_off(p.ql, k0 + d), kPkLoadStream);
        b.w[d][0] = v[0];
        b.w[d][1] = v[1];
      } else {
        b.w[d][0] = __builtin_amdgcn_raw_buffer_load_b32(rq, q_voff, qrow_off(p.ql, k0 + d), kPkLoadStream);
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) b.x[mb] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[mb], k0 * 2, 0);
  };

  // accL / accR: byte b (columns 2b, 2b + 1 of the lane) masked low nibble / both nibbles
  pk_f4 accL[MB][CPL / 2], accR[MB][CPL / 2], off[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    off[mb] = pk_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < CPL / 2; ++b) accL[mb][b] = accR[mb][b] = off[mb];
  }
  const pk_u4v eight_u = {0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u};
  const pk_half8 eight = __builtin_bit_cast(pk_half8, eight_u);

  auto compute = [&](const SkStep<MB, WPL>& b) {
    pk_half8 xa[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xa[mb] = __builtin_bit_cast(pk_half8, b.x[mb]);
      off[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mb], eight, off[mb], 0, 0, 0);
    }
#pragma unroll
    for (int wi = 0; wi < WPL; ++wi) {
      uint32_t wx[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) wx[d] = b.w[d][wi] ^ 0x88888888u;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + bb) << 16) | (uint32_t)bb;
        pk_u4v raw, lo;
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) {
          raw[dd] = __builtin_amdgcn_perm(wx[2 * dd + 1], wx[2 * dd], sel);
          lo[dd] = raw[dd] & 0x000f000fu;
        }
        const int by = 4 * wi + bb;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          accL[mb][by] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mb], __builtin_bit_cast(pk_half8, lo), accL[mb][by], 0, 0, 0);
          accR[mb][by] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mb], __builtin_bit_cast(pk_half8, raw), accR[mb][by], 0, 0, 0);
        }
      }
    }
  };

  // ---- per column: remove the +8 offset, apply 2^24 / 2^20 and the group scale ------------
  // acc[mb][c] holds rows m0 + mb*16 + 4g + r of the lane's column c.
  pk_f4 acc[MB][CPL];
  auto fold = [&](bool first) {
    float sc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      float sv = 1.0f;
      if constexpr (HAS_GS) {
        const uint32_t word = sraw[c >> 3][(c & 7) >> 1];
        sv = (float)__builtin_bit_cast(pk_half, (uint16_t)((c & 1) ? (word >> 16) : (word & 0xffffu)));
      }
      sc[c] = sv * ((c & 1) ? 1048576.0f : 16777216.0f);
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int by = 0; by < CPL / 2; ++by) {
        const pk_f4 lo = (accL[mb][by] - off[mb]) * sc[2 * by];
        const pk_f4 hi = (accR[mb][by] - accL[mb][by] - off[mb] * 16.0f) * sc[2 * by + 1];
        acc[mb][2 * by] = first ? lo : acc[mb][2 * by] + lo;
        acc[mb][2 * by + 1] = first ? hi : acc[mb][2 * by + 1] + hi;
      }
  };

  // ---- k-steps: a ring of PD buffers, each refilled PD steps ahead -----------------------
  SkStep<MB, WPL> ring[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i)
    if (i < nsteps) load(ring[i], i);
  if constexpr (MG) {
    // 128-row groups of 4 k-steps (the plan makes the wave's rows a whole number of them);
    // at each boundary the group's sums are scaled into acc and the accumulators restart,
    // while the ring's loads for the next group stay in flight.
    static_assert(HAS_GS && PD <= 4 && 4 % PD == 0, "MG: whole groups of 4 k-steps");
    const int groups = nsteps >> 2;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[mb][c] = pk_f4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int gi = 0; gi < groups; ++gi) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int s = 4 * gi + i;
        compute(ring[i % PD]);
        if (s + PD < nsteps) load(ring[i % PD], s + PD);
      }
      mfma_drain();
      fold(gi == 0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        off[mb] = pk_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < CPL / 2; ++b) accL[mb][b] = accR[mb][b] = off[mb];
      }
      if (gi + 1 < groups) {
        const int srow = (kb / p.group + gi + 1) * p.N * 2;
#pragma unroll
        for (int i = 0; i < WPL; ++i)
          sraw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, word0 * 16 + 16 * i, srow, kPkLoadStream);
      }
    }
  } else {
    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
      for (int i = 0; i < PD; ++i) {
        const int s = s0 + i;
        if (s < nsteps) {
          compute(ring[i]);
          if (s + PD < nsteps) load(ring[i], s + PD);
        }
      }
    }
    mfma_drain();
    fold(true);
  }

  // ---- add the waves' tiles in LDS: waves NB.. store, waves 0..NB-1 add their own, and the
  // buffers are summed in a fixed order: 4 waves ((w2 + w0) + (w3 + w1)); 8 waves
  // ((w4 + w0) + (w6 + w2)) + ((w5 + w1) + (w7 + w3)) ----------------------------------
  __shared__ float red[NB][MB * 16][TC + kSkPad];
  auto tile_vec = [&](int mb, int r, int c4) {
    return pk_f4{acc[mb][4 * c4][r], acc[mb][4 * c4 + 1][r], acc[mb][4 * c4 + 2][r],
                 acc[mb][4 * c4 + 3][r]};
  };
  if (wave >= NB) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c4 = 0; c4 < CPL / 4; ++c4)
          *reinterpret_cast<pk_f4*>(&red[wave - NB][mb * 16 + 4 * g + r][CPL * j + 4 * c4]) =
              tile_vec(mb, r, c4);
  }
  __syncthreads();
  if (wave < NB) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c4 = 0; c4 < CPL / 4; ++c4) {
          pk_f4* q = reinterpret_cast<pk_f4*>(&red[wave][mb * 16 + 4 * g + r][CPL * j + 4 * c4]);
          *q = *q + tile_vec(mb, r, c4);
        }
  }
  __syncthreads();
  const int rows = min(MB * 16, p.M - m0);
  if constexpr (L2) {
    // Quads of 4 columns, QPT per thread: this slice's partial block, then (last workgroup of
    // the tile) the slices' sum in slice order.
    constexpr int QPR = TC / 4;  // quads per row
    constexpr int QPT = MB * 16 * QPR / (64 * NW);
    static_assert(QPT >= 1 && (MB * 16 * QPR) % (64 * NW) == 0, "quads per thread");
    const int64_t plane = (int64_t)p.M * p.npad;
    float* const blk = p.partials + (int64_t)m0 * p.npad + tile * TC;
    pk_f4 own[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int qi = t + i * 64 * NW, m = qi / QPR, c4 = (qi % QPR) * 4;
      auto rq = [&](int nb) { return *reinterpret_cast<const pk_f4*>(&red[nb][m][c4]); };
      if constexpr (NB == 2) own[i] = rq(0) + rq(1);
      else own[i] = (rq(0) + rq(2)) + (rq(1) + rq(3));
      if (m < rows) *reinterpret_cast<pk_f4*>(blk + slice * plane + (int64_t)m * p.npad + c4) = own[i];
    }
    if (!splitk_arrive(p.counters + 32 * (tile * p.row_parts + part), p.split)) return;
    // The gather: QG quads' loads of up to 8 slices each go out together, so a thread waits
    // for one memory round trip per 8 slices, not one per quad (measured on MI355X, qkv and
    // o_proj at M = 32: 1-2% faster end to end); each quad is summed in slice order, the
    // arithmetic of splitk_reduce_kernel. Quads past the rows or columns load row 0 of the
    // block (in bounds) and are not stored.
    constexpr int QG = QPT < 2 ? QPT : 2;
#pragma unroll
    for (int i0 = 0; i0 < QPT; i0 += QG) {
      pk_f4 v[QG];
      const float* src[QG];
      bool ok[QG];
#pragma unroll
      for (int q = 0; q < QG; ++q) {
        const int qi = t + (i0 + q) * 64 * NW, m = qi / QPR, c4 = (qi % QPR) * 4;
        ok[q] = m < rows && tile * TC + c4 < p.N;
        src[q] = blk + (int64_t)(ok[q] ? m : 0) * p.npad + c4;
        v[q] = own[i0 + q];
      }
      for (int s0 = 0; s0 < p.split; s0 += 8) {
        pk_f4 pv[QG][8];
#pragma unroll
        for (int q = 0; q < QG; ++q)
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int sl = min(s0 + u, p.split - 1);
            pv[q][u] = sl == slice ? own[i0 + q] : *reinterpret_cast<const pk_f4*>(src[q] + sl * plane);
          }
#pragma unroll
        for (int q = 0; q < QG; ++q)
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (s0 + u == 0) v[q] = pv[q][0];
            else if (s0 + u < p.split) v[q] += pv[q][u];
          }
      }
#pragma unroll
      for (int q = 0; q < QG; ++q) {
        if (!ok[q]) continue;
        const int qi = t + (i0 + q) * 64 * NW, m = qi / QPR, c4 = (qi % QPR) * 4;
        const int col = tile * TC + c4;
        const int64_t o = (int64_t)(m0 + m) * p.ldc + col;
        const pk_f4 w = p.epi(v[q], col);
#pragma unroll
        for (int e = 0; e < 4; ++e) store_from_f32(p.c, p.c_dtype, o + e, w[e]);
      }
    }
    return;
  }
  if (p.split > 1) {
    // fp32 partials for the reduce launch: quads of 4 columns (N % 16 == 0, so a quad is all
    // in or all out), stored non-temporally -- they are read once, by another kernel
    // (measured on the Llama-3-8B layers: M = 32 and 64 rows 5-19% faster than element stores
    // through the cache)
    constexpr int QPR = TC / 4;
    for (int qi = t; qi < rows * QPR; qi += 64 * NW) {
      const int m = qi / QPR, c4 = (qi % QPR) * 4;
      const int col = tile * TC + c4;
      if (col >= p.N) continue;
      auto rq = [&](int nb) { return *reinterpret_cast<const pk_f4*>(&red[nb][m][c4]); };
      pk_f4 v;
      if constexpr (NB == 2) v = rq(0) + rq(1);
      else v = (rq(0) + rq(2)) + (rq(1) + rq(3));
      __builtin_nontemporal_store(v, reinterpret_cast<pk_f4*>(p.partials + ((int64_t)slice * p.M + m0 + m) * p.N + col));
    }
    return;
  }
  for (int idx = t; idx < rows * TC; idx += 64 * NW) {
    const int m = idx / TC, cl = idx % TC;
    const int col = tile * TC + cl;
    if (col >= p.N) continue;
    float v;
    if constexpr (NB == 2) v = red[0][m][cl] + red[1][m][cl];
    else v = (red[0][m][cl] + red[2][m][cl]) + (red[1][m][cl] + red[3][m][cl]);
    store_from_f32(p.c, p.c_dtype, (int64_t)(m0 + m) * p.ldc + col, p.epi(v, col));
  }
}

// ---------------------------------------------------------------------------------------
// Planning and launch.
// ---------------------------------------------------------------------------------------
// Waves the automatic plan aims for: the fewest slices whose workgroups reach this many waves
// (about 1.5 per SIMD) won on every Llama-3-8B layer at M = 8..64 (MI355X): fewer waves
// leave HBM requests short, more slices add fp32 partials.
constexpr int kSkWaveTarget = 1536;

// The plan for nw waves per workgroup, cpl_fixed columns per lane (0: chosen here).
static bool skinny_plan_nw(int M, int N, int K, int group, bool has_gs, int split_req, int nw,
                           int cpl_fixed, SkinnyPlan* out) {
  // 16 columns per lane (256-column tiles) hold at most two 16-row blocks; 8 columns per lane
  // (128-column tiles) up to four, with two row parts above 64 rows.
  const int mb = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const int rp = (int)cdiv(M, mb * 16);
  // A wave takes k_slice / nw rows, a multiple of the 32-row k-step lying in one group; with
  // two 16-row blocks and 8 columns per lane (the registers for a second set of sums), also a
  // whole number of 128-row groups, folded at each boundary -- half the slices of down and
  // gate_up at M = 32 (measured on MI355X: 22.6 -> 18.5 and 19.3 -> 17.8 us with group-256
  // weights, which take those slices without folds).
  const bool mg_ok = has_gs && group == 128 && mb == 2;
  auto ok = [&](int s, int cpl) {
    if (s < 1 || K % s || (K / s) % (nw * kSkStep)) return false;
    const int rows_w = K / s / nw;
    return !has_gs || group % rows_w == 0 || (mg_ok && cpl == 8 && rows_w % group == 0);
  };
  auto waves = [&](int cpl, int s) {
    return (int64_t)cdiv(N, 16 * cpl) * rp * s * nw;
  };
  auto pick = [&](int cpl) {  // fewest slices reaching the wave target, else the most
    int last = 0;
    for (int s = 1; s <= K / (nw * kSkStep); ++s)
      if (ok(s, cpl)) {
        last = s;
        if (waves(cpl, s) >= kSkWaveTarget) return s;
      }
    return last;
  };
  int cpl = 8, split = 0;
  if (split_req > 0) {
    if (cpl_fixed) cpl = cpl_fixed;
    else if (M <= 32 && waves(16, split_req) >= kSkWaveTarget && ok(split_req, 16)) cpl = 16;
    if (!ok(split_req, cpl)) return false;
    split = split_req;
  } else if (cpl_fixed) {
    cpl = cpl_fixed;
    split = pick(cpl);
  } else {
    // 256-column tiles when they reach the wave target without extra slices, unless
    // group-spanning waves on 128-column tiles need fewer slices
    int first = 0;
    for (int s = 1; s <= K / (nw * kSkStep) && !first; ++s)
      if (ok(s, 16)) first = s;
    const int s8 = pick(8);
    if (first && M <= 32 && waves(16, first) >= kSkWaveTarget && !(mg_ok && s8 && s8 < first)) {
      cpl = 16;
      split = first;
    } else {
      split = s8;
    }
  }
  if (!split) return false;
  *out = {mb, cpl, nw, rp, split, K / split, (int)cdiv(N, 16 * cpl),
          has_gs && K / split / nw > group};
  return true;
}

// Fixed layout: 0 = automatic, else (cpl << 8) | nw. -1: not yet read from the environment.
static std::atomic<int> g_skinny_layout{-1};

static int skinny_layout_get() {
  int v = g_skinny_layout.load(std::memory_order_acquire);
  if (v >= 0) return v;
  int c = 0, w = 0, env = 0;
  if (const char* e = getenv("PK_SKINNY_CFG"))
    if (sscanf(e, "%d,%d", &c, &w) == 2 && (c == 8 || c == 16) && (w == 4 || w == 8))
      env = (c << 8) | w;
  int expected = -1;  // a concurrent setter wins
  g_skinny_layout.compare_exchange_strong(expected, env, std::memory_order_acq_rel);
  return g_skinny_layout.load(std::memory_order_acquire);
}

bool skinny_layout_set(int cpl, int nw) {
  if (cpl == 0 && nw == 0) {
    g_skinny_layout.store(0, std::memory_order_release);
    return true;
  }
  if (!((cpl == 8 || cpl == 16) && (nw == 4 || nw == 8))) return false;
  g_skinny_layout.store((cpl << 8) | nw, std::memory_order_release);
  return true;
}

bool skinny_plan(int M, int N, int K, int group, bool has_gs, int split_req, SkinnyPlan* out,
                 bool tiled) {
  if (M < kSkinnyMinM || M > kSkinnyMaxM || N % 16 || K % 128) return false;
  // Above 64 rows every weight is read by two row parts; that beat the LDS-tiled GEMM only
  // on layers of at most 4096 x 4096 weights (measured at M = 96 and 128).
  if (M > 64 && (int64_t)K * N > 4096ll * 4096) return false;
  // A fixed layout (columns per lane, waves per workgroup), set through
  // pk_w4a16_skinny_layout; the environment variable PK_SKINNY_CFG="cpl,nw" sets it once per
  // process, at the first plan.
  const int cfg = skinny_layout_get();
  if (cfg) {
    const int c = cfg >> 8, w = cfg & 0xff;
    return skinny_plan_nw(M, N, K, group, has_gs, split_req, w, M > 32 ? 8 : c, out);
  }
  // 8 waves (half the slices for the same waves in flight); 4 where slices of 8 k-steps do
  // not fit K, the group or the requested split. Block-layout weights with one 16-row block:
  // 128-column tiles, whose two halves of each 256-byte block row go to two workgroups of one
  // XCD (faster there on the larger layers; 256-column tiles on the row layout).
  const int c = tiled && M <= 16 ? 8 : 0;
  return skinny_plan_nw(M, N, K, group, has_gs, split_req, 8, c, out) ||
         skinny_plan_nw(M, N, K, group, has_gs, split_req, 4, c, out);
}

// Buffer offsets are 32-bit: weights, scales and activations must each stay below 2 GiB.
bool skinny_fits(int M, int N, int K, int64_t lda, int64_t ldq, int group, bool has_gs) {
  return (int64_t)K * ldq * 4 < (1ll << 31) && (int64_t)M * lda * 2 < (1ll << 31) &&
         (!has_gs || (int64_t)(K / group) * N * 2 < (1ll << 31));
}

template <int MB, int CPL, int NW, bool GS, bool MG>
static void launch_skinny_t(const SkinnyParams& p, bool l2, hipStream_t s) {
  // k-steps in flight per wave, measured on the Llama-3-8B shapes: 3 for one 16-row block of
  // 16 columns per lane (162 VGPRs, three waves per SIMD; 2-3% faster than 4 at two waves),
  // 2 for two blocks; 8 columns per lane halve the weight registers. Group-spanning waves
  // keep a divisor of the group's 4 k-steps.
  constexpr int PD = MG ? 2 : CPL == 16 ? (MB == 1 ? 3 : 2) : (MB == 1 ? 4 : MB == 2 ? 3 : 2);
  constexpr int OCC = NW == 4 ? 2 : 1;
  // tiles rounded up to whole groups of 8 XCDs (of pairs with 8 columns per lane)
  const unsigned slots = (unsigned)(cdiv(p.tiles, CPL == 8 ? 16 : 8) * (CPL == 8 ? 16 : 8));
  if (l2) {
    w4a16_skinny_kernel<MB, CPL, NW, GS, PD, OCC, true, MG>
        <<<slots * p.split * p.row_parts, 64 * NW, 0, s>>>(p);
    return;
  }
  w4a16_skinny_kernel<MB, CPL, NW, GS, PD, OCC, false, MG>
      <<<dim3(slots * p.row_parts, p.split), 64 * NW, 0, s>>>(p);
}

template <int MB, int CPL, bool GS, bool MG = false>
static void launch_skinny_nw(const SkinnyParams& p, int nw, bool l2, hipStream_t s) {
  if (nw == 8) launch_skinny_t<MB, CPL, 8, GS, MG>(p, l2, s);
  else launch_skinny_t<MB, CPL, 4, GS, MG>(p, l2, s);
}

template <bool GS>
static void launch_skinny_cfg(const SkinnyPlan& pl, const SkinnyParams& p, bool l2, hipStream_t s) {
  if (pl.cpl == 16) {
    if (pl.mb == 1) launch_skinny_nw<1, 16, GS>(p, pl.nw, l2, s);
    else launch_skinny_nw<2, 16, GS>(p, pl.nw, l2, s);
  } else {
    if (pl.mb == 1) launch_skinny_nw<1, 8, GS>(p, pl.nw, l2, s);
    else if (pl.mb == 2) {
      if constexpr (GS) {
        if (pl.mg) return launch_skinny_nw<2, 8, GS, true>(p, pl.nw, l2, s);
      }
      launch_skinny_nw<2, 8, GS>(p, pl.nw, l2, s);
    }
    else launch_skinny_nw<4, 8, GS>(p, pl.nw, l2, s);
  }
}

// The split-K slices hand off through L2 in the launch (no reduce launch) for one 16-row
// block, and for two on layers of at most 4096 x 6144 weights. Measured on the Llama-3-8B
// layers (graphs over rotating weights): M = 8 gains about 1 us on every layer (qkv 11.3 ->
// 10.3, o_proj 9.4 -> 8.2, gate_up 15.1 -> 14.3, down 15.9 -> 14.8 us); at M = 32 the last
// workgroup's gather of 32 * split partial rows per tile pays on the smaller layers (qkv
// 13.85 -> 13.1, o_proj 12.1 -> 10.6 us) but not on the larger (gate_up 22.1 -> 22.8, down
// 22.7 -> 26.1), and with four blocks it was slower everywhere, so those keep the reduce
// launch. Group-spanning plans (half the slices, 128-column tiles) gather a quarter of those
// bytes per tile and hand off in L2 on every layer (down M = 32 with 7 slices: 19.5 -> 18.5).
bool skinny_l2(const SkinnyPlan& pl, bool l2) {
  const int64_t weights = (int64_t)pl.split * pl.k_slice * pl.tiles * 16 * pl.cpl;
  const bool blocks_ok = pl.mb == 1 || (pl.mb == 2 && (weights <= 4096ll * 6144 || pl.mg));
  return pl.split > 1 && blocks_ok && pl.tiles * pl.row_parts <= kWsMaxTiles && l2;
}

size_t skinny_workspace_bytes(const SkinnyPlan& pl, int M, int N) {
  if (pl.split <= 1) return 0;
  const size_t flat = (size_t)pl.split * M * N * sizeof(float);
  const size_t padded = (size_t)pl.split * M * pl.tiles * 16 * pl.cpl * sizeof(float);
  return kWsCounterBytes + (flat > padded ? flat : padded);
}

int skinny_launch(const SkinnyPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                  int64_t ldq, const void* scales, int group, OutEpi epi, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                  bool partials_only, bool tiled) {
  if (tiled && N % 256) {
    set_error("w4a16 skinny: block-layout weights need N %% 256 == 0");
    return PK_EUNSUPPORTED;
  }
  SkinnyParams p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.qw = qw;
  p.ldq = ldq;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = scales ? group : K;
  p.epi = epi;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.split = pl.split;
  p.k_slice = pl.k_slice;
  p.tiles = pl.tiles;
  p.row_parts = pl.row_parts;
  p.partials = pl.split > 1 ? split_partials(workspace, partials_only) : nullptr;
  p.counters = ws_counters(workspace);
  p.npad = pl.tiles * 16 * pl.cpl;
  p.ql = qlayout(tiled, ldq, N);
  const bool l2 = !partials_only && pl.split > 1 && skinny_l2(pl, splitk_in_l2_ok(s));
  if (scales) launch_skinny_cfg<true>(pl, p, l2, s);
  else launch_skinny_cfg<false>(pl, p, l2, s);
  PK_LAUNCH_CHECK("w4a16 skinny");
  if (pl.split > 1 && !partials_only && !l2)
    return splitk_reduce(p.partials, pl.split, M, N, epi, c, c_dtype, ldc, s, true);
  return PK_OK;
}

}  // namespace pk
