// W4A16 matmul for 5 <= M <= 32 activation rows: the HBM-bound middle between the GEMV
// (M <= 4) and the LDS-tiled GEMM. C = tensor_scale * A (M, K) fp16 @ deq(W) (K, N), with W in
// the packed layout of gemm_int4.pack_int4_n (gemm_int4.py:65-72) viewed as int32 words
// (word j of row k = columns 8j..8j+7, nibble i = column 8j+i) and the group scales of
// quantize.rtn_layer along K (quantize.py:63-68).
//
// Work decomposition: grid.x = column tiles of 256 columns (128 bytes of every row),
// grid.y = split-K slices of k_slice rows (contiguous, as gemm_splitk.py:49-53). The 4 waves
// of a workgroup take consecutive quarters of the slice; a wave walks its rows in k-steps of
// 32 with several k-steps of loads in flight (no LDS staging: weights go straight to
// registers).
//
// Per k-step a lane (j = lane % 16, g = lane / 16) loads 8 bytes (16 columns 16j..16j+15) of
// the 8 rows 8g..8g+7, plus 16 bytes of activations (row j of a 16-row block, the same 8 k).
// That is exactly the operand layout of v_mfma_f32_16x16x32_f16: lane L supplies A[L%16][8g+d]
// and B[8g+d][L%16] for d = 0..7, so MFMA number c (c = 0..15) multiplies the activations by
// weight column 16j + c of lane j, and the 16 x 16 result lands in lane L as rows 4g..4g+3 of
// column 16j + c. No data crosses lanes.
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
// at the end (exact powers of two folded into the scale).
//
// Reduction: the 4 waves' tiles are added in LDS in a fixed order, ((w2 + w0) + (w3 + w1));
// with split-K every slice writes (split, M, N) fp32 partials and splitk_reduce_kernel adds
// them in slice order, so results are bitwise reproducible. (Adding the slices through one
// XCD's L2 inside this kernel, as the M <= 4 GEMV does, was measured slower here for every
// split: the last workgroup of a tile has M * split partials per thread to gather.)
#include "pk_internal.h"

namespace pk {

constexpr int kSkTileCols = 256;  // columns per workgroup tile (16 lanes x 16 columns)
constexpr int kSkStep = 32;       // rows per k-step (4 lane groups x 8 rows)
constexpr int kSkPad = 4;         // LDS row padding (floats)

struct SkinnyParams {
  const pk_half* a;
  int64_t lda;
  const uint32_t* qw;
  int64_t ldq;
  const pk_half* scales;  // (K/G, N) or null
  int group;
  float tensor_scale;
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int split, k_slice;
  float* partials;  // (split, M, N) fp32 when split > 1
};

template <int MB>
struct SkStep {
  pk_u2v w[8];   // rows 8g..8g+7, words 2j', 2j'+1 of the tile
  pk_u4v x[MB];  // activations: row j of each 16-row block, k = 8g..8g+7
};

template <int MB, bool HAS_GS, int PD, int OCC>
__global__ __launch_bounds__(256, OCC) void w4a16_skinny_kernel(SkinnyParams p) {
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x, slice = blockIdx.y;
  const int words_total = p.N >> 3;
  // The ragged last tile re-reads in-bounds words; those columns are never stored.
  const int word0 = min(tile * (kSkTileCols / 8) + 2 * j, words_total - 2);
  const int rows_w = p.k_slice >> 2;
  const int nsteps = rows_w / kSkStep;
  const int kb = slice * p.k_slice + wave * rows_w;

  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.qw, (uint32_t)((int64_t)p.K * p.ldq * 4));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(HAS_GS ? (const void*)p.scales : (const void*)p.qw,
                HAS_GS ? (uint32_t)((int64_t)(p.K / p.group) * p.N * 2) : 0u);
  const int ldq4 = (int)p.ldq * 4;
  const int q_voff = 8 * g * ldq4 + word0 * 4;
  int a_voff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) a_voff[mb] = (int)(min(mb * 16 + j, p.M - 1) * p.lda + 8 * g) * 2;
  // The wave's rows lie in group kb / group: its 16 column scales, requested first.
  pk_u4v sraw[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if constexpr (HAS_GS) {
    const int srow = (kb / p.group) * p.N * 2;
    sraw[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, word0 * 16, srow, 0);
    sraw[1] = __builtin_amdgcn_raw_buffer_load_b128(rs, word0 * 16 + 16, srow, 0);
  }

  auto load = [&](SkStep<MB>& b, int s) {
    const int k0 = kb + s * kSkStep;
#pragma unroll
    for (int d = 0; d < 8; ++d) b.w[d] = __builtin_amdgcn_raw_buffer_load_b64(rq, q_voff, (k0 + d) * ldq4, 0);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) b.x[mb] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[mb], k0 * 2, 0);
  };

  // accL / accR: byte b (columns 16j + 2b, 16j + 2b + 1) masked low nibble / both nibbles
  pk_f4 accL[MB][8], accR[MB][8], off[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    off[mb] = pk_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < 8; ++b) accL[mb][b] = accR[mb][b] = off[mb];
  }
  const pk_u4v eight_u = {0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u};
  const pk_half8 eight = __builtin_bit_cast(pk_half8, eight_u);

  auto compute = [&](const SkStep<MB>& b) {
    pk_half8 xa[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xa[mb] = __builtin_bit_cast(pk_half8, b.x[mb]);
      off[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mb], eight, off[mb], 0, 0, 0);
    }
#pragma unroll
    for (int wi = 0; wi < 2; ++wi) {
      uint32_t wx[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const pk_u2v wd = b.w[d];
        wx[d] = wd[wi] ^ 0x88888888u;
      }
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

  // ---- k-steps: a ring of PD buffers, each refilled PD steps ahead -----------------------
  SkStep<MB> ring[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i)
    if (i < nsteps) load(ring[i], i);
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

  // ---- per column: remove the +8 offset, apply 2^24 / 2^20 and the group scale ------------
  // acc[mb][c] holds rows mb*16 + 4g + r of column 16j + c.
  pk_f4 acc[MB][16];
  {
    float sc[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
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
      for (int by = 0; by < 8; ++by) {
        acc[mb][2 * by] = (accL[mb][by] - off[mb]) * sc[2 * by];
        acc[mb][2 * by + 1] = (accR[mb][by] - accL[mb][by] - off[mb] * 16.0f) * sc[2 * by + 1];
      }
  }

  // ---- add the 4 waves' tiles in LDS: ((w2 + w0) + (w3 + w1)) ---------------------------
  __shared__ float red[2][MB * 16][kSkTileCols + kSkPad];
  if (wave >= 2) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const pk_f4 v = {acc[mb][4 * c4][r], acc[mb][4 * c4 + 1][r], acc[mb][4 * c4 + 2][r],
                           acc[mb][4 * c4 + 3][r]};
          *reinterpret_cast<pk_f4*>(&red[wave - 2][mb * 16 + 4 * g + r][16 * j + 4 * c4]) = v;
        }
  }
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          pk_f4* q = reinterpret_cast<pk_f4*>(&red[wave][mb * 16 + 4 * g + r][16 * j + 4 * c4]);
          const pk_f4 v = {acc[mb][4 * c4][r], acc[mb][4 * c4 + 1][r], acc[mb][4 * c4 + 2][r],
                           acc[mb][4 * c4 + 3][r]};
          *q = *q + v;
        }
  }
  __syncthreads();
  const int col = tile * kSkTileCols + t;
  if (col < p.N) {
    for (int m = 0; m < p.M; ++m) {
      const float v = red[0][m][t] + red[1][m][t];
      if (p.split == 1)
        store_from_f32(p.c, p.c_dtype, (int64_t)m * p.ldc + col, v * p.tensor_scale);
      else
        p.partials[((int64_t)slice * p.M + m) * p.N + col] = v;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Planning and launch.
// ---------------------------------------------------------------------------------------
bool skinny_plan(int M, int N, int K, int group, bool has_gs, int split_req, SkinnyPlan* out) {
  if (M < kSkinnyMinM || M > kSkinnyMaxM || N % 16 || K % 128) return false;
  // A wave takes k_slice / 4 rows, a multiple of the 32-row k-step lying in one group.
  auto ok = [&](int s) {
    if (s < 1 || K % s || (K / s) % 128) return false;
    const int rows_w = K / s / 4;
    return !has_gs || group % rows_w == 0;
  };
  int split = 0;
  if (split_req > 0) {
    if (!ok(split_req)) return false;
    split = split_req;
  } else {
    // fp32 partials cost 8*S*M*N bytes of traffic against K*N/2 of weights: 8 slices
    // (measured fastest on MI355X for M = 8..32 against 16 and 32 on the Llama-3-8B shapes), or
    // the nearest count that satisfies the group constraint (more slices first, since short
    // slices are what long K needs).
    const int base = 8;
    for (int s = base; s <= K / 128 && !split; ++s)
      if (ok(s)) split = s;
    for (int s = min(base - 1, K / 128); s >= 1 && !split; --s)
      if (ok(s)) split = s;
    if (!split) return false;
  }
  *out = {M <= 16 ? 1 : 2, split, K / split, (int)cdiv(N, kSkTileCols)};
  return true;
}

// Buffer offsets are 32-bit: weights, scales and activations must each stay below 2 GiB.
bool skinny_fits(int M, int N, int K, int64_t lda, int64_t ldq, int group, bool has_gs) {
  return (int64_t)K * ldq * 4 < (1ll << 31) && (int64_t)M * lda * 2 < (1ll << 31) &&
         (!has_gs || (int64_t)(K / group) * N * 2 < (1ll << 31));
}

template <int MB, bool GS>
static void launch_skinny_t(const SkinnyParams& p, int tiles, hipStream_t s) {
  // k-steps in flight per wave, measured on the Llama-3-8B shapes: 3 for one 16-row block
  // (162 VGPRs, three waves per SIMD; 2-3% faster than 4 at two waves), 2 for two blocks.
  constexpr int PD = MB == 1 ? 3 : 2;
  w4a16_skinny_kernel<MB, GS, PD, 2><<<dim3(tiles, p.split), 256, 0, s>>>(p);
}

int skinny_launch(const SkinnyPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                  int64_t ldq, const void* scales, int group, float tensor_scale, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                  bool partials_only) {
  SkinnyParams p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.qw = qw;
  p.ldq = ldq;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = scales ? group : K;
  p.tensor_scale = tensor_scale;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.split = pl.split;
  p.k_slice = pl.k_slice;
  p.partials = pl.split > 1 ? split_partials(workspace, partials_only) : nullptr;
  const bool gs = scales != nullptr;
  if (pl.mb == 1) {
    if (gs) launch_skinny_t<1, true>(p, pl.tiles, s);
    else launch_skinny_t<1, false>(p, pl.tiles, s);
  } else {
    if (gs) launch_skinny_t<2, true>(p, pl.tiles, s);
    else launch_skinny_t<2, false>(p, pl.tiles, s);
  }
  PK_LAUNCH_CHECK("w4a16 skinny");
  if (pl.split > 1 && !partials_only)
    return splitk_reduce(p.partials, pl.split, M, N, tensor_scale, c, c_dtype, ldc, s);
  return PK_OK;
}

}  // namespace pk
