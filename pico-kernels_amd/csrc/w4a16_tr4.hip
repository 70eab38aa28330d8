// W4A16 GEMM for large M on gfx950 with the int4 weights kept packed in LDS
// (gemm_int4.py:21-55 is the operation: C = A @ dequant(B), B int4 codes packed 8 per int32
// along N as pack_int4_n writes them (gemm_int4.py:65-72), optional fp16 group scales along K).
//
// Shape: 128 x 256 workgroup tiles (64 x 256 up to 128 rows of activations), BK = 128, eight
// waves. Wave w owns output columns 64 (w % 4) .. +63 of all the tile's rows and k half
// h = w / 4 of every k-tile: waves w and w + 4 run
// on the same SIMD, compute the same 128 x 64 block over different k and add their
// accumulators once, at the end. So each SIMD has two independent instruction streams (one
// covers the other's LDS and dependency waits) while its per-tile work -- MFMAs, LDS reads,
// and the dequantisation of each weight exactly once -- is what one wave of a 4-wave 128 x 64
// layout would do. v_mfma_f32_32x32x16_f16 with B as the first operand (each accumulator is
// C^T: register 4 q + e of lane l is row l % 32, column 8 q + 4 (l / 32) + e of a 32 x 32
// fragment), 4 x 2 fragments per wave.
//
//  * A (M, K) fp16, the packed B words and the group scales go global -> LDS by buffer DMA
//    (buffer_load ... lds), no VGPR staging; three stages of 49 KB.
//    A rows are 256 bytes (128 k), 16-byte chunk c of row r in slot c ^ (r & 15): the 16 rows
//    a 16-lane group reads at one chunk cover all 64 banks.
//    B rows are the 128 bytes of 256 packed columns at one k, chunk c of k-row r in slot
//    c ^ ((r >> 1) & 7) ^ 4 ((r >> 4) & 1).
//  * B leaves LDS through ds_read_b64_tr_b4: within each 16-lane group, lane q receives nibble q
//    (column q of an 8-byte, 16-column segment) of the rows the group's 16 lanes address, one
//    row per result nibble (measured on MI355X). For a 32 x 32 x 16 step the lanes of group g
//    hold columns 16 (g & 1) + q at k 8 (g >> 1) .. +7; lane 16 g + e addresses k row
//    16 (2 p + e / 8) + 8 (g >> 1) + pi(e % 8) of its half, pi = (0 2 4 6 1 3 5 7), so one read
//    gives a lane the codes of k-steps 2p and 2p+1 in an order from which plain masks extract
//    (k, k+1) pairs:
//      d & 0x000F000F -> nibbles 0, 4 = (k0, k1) in the mantissas of 1024 + u,
//      d & 0x00F000F0 -> nibbles 1, 5 = (k2, k3) in the mantissas of   64 + u,
//    and the same on d >> 8 for (k4, k5), (k6, k7), with u = code + 8: one AND-XOR each
//    ((x ^ 8) | 0x6400 = (x & 0xF) ^ 0x6408). Subtracting 1032 (72) gives the exact code,
//    times the fp16 group scale the product is rounded once, as the other W4A16 GEMMs here do.
//  * Per k-tile: the waves meet at one barrier (tile t landed in every wave, tile t-1 read by
//    all), the DMA of tile t+2 goes into tile t-1's stage, then each wave reads its k half's B
//    codes, scales and A fragments and runs its four k-steps, the next step's A fragments read
//    and B dequantised between the current step's MFMAs.
//  * Epilogue: the k-half-1 waves leave their accumulators in LDS; the k-half-0 waves add
//    them, scale, convert, stage slices and store whole lines.
//
//  * Split-K: workgroup (tile, slice) runs k-tiles slice * K / (128 S) .. and stores its fp32
//    partial plane; a fixed-order reduce adds the S planes (for shapes whose tiles alone
//    leave CUs idle).
//
// Requires N % 256 == 0, K % 128 S == 0, a group size that is a multiple of 64 (or
// per-tensor), 16-byte aligned A rows and output rows, and buffers addressable with 32-bit
// offsets. Rows past M are clamped to row M-1 for loading and never stored.
#include "pk_internal.h"

namespace pk {

#define PK_LDS(p) ((__attribute__((address_space(3))) void*)(p))
typedef int pk_v2i __attribute__((ext_vector_type(2)));

struct Tr4Params {
  const pk_half* a;
  int64_t lda;            // elements
  const uint32_t* b;      // int4 words (K, N / 8)
  int64_t ldb;            // words
  const pk_half* scales;  // (K / group, N) or null
  int group;
  OutEpi epi;             // epilogue: tensor scale and optional bias
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
  int kt_slice;     // k-tiles per split-K slice (all of K when unsplit)
  int64_t c_slice;  // elements between the slices' outputs (fp32 partial planes)
  QLayout ql;       // where the weight words live
};

// global -> LDS DMA, 16 or 4 bytes per lane (lane L writes lds + 16 L / lds + 4 L)
__device__ __forceinline__ void tr4_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS(lds), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void tr4_dma4(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS(lds), 4, voff, soff, 0, 0);
}

// Slot of 16-byte chunk c of A row r / of B k-row r.
__device__ __forceinline__ int tr4_aslot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int tr4_bslot(int r, int c) { return c ^ ((r >> 1) & 7) ^ (((r >> 4) & 1) << 2); }

__device__ __forceinline__ pk_half2 tr4_h2(uint32_t v) { return __builtin_bit_cast(pk_half2, v); }

// XCD-aware tile order: consecutive logical tiles on one XCD, walked 4 tile rows deep.
__device__ __forceinline__ void tr4_tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
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

// s_waitcnt immediate for vmcnt(v) alone.
constexpr int tr4_wait_vm(int v) { return (v & 15) | (7 << 4) | (15 << 8) | ((v >> 4) << 14); }

template <bool GS, int BM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void w4a16_tr4_kernel(Tr4Params p) {
  static_assert(BM == 128 || BM == 64, "tiles of 128 or 64 rows");
  constexpr int BN = 256, WN = 64;
  constexpr int FM = BM / 32, FN = 2;  // 32 x 32 fragments per wave
  constexpr int A_DMA = BM / 32;       // BM x 256 bytes of A per tile: A_DMA x 1 KB per wave
  constexpr int B_DMA = 2;       // 16 KB of packed B per tile: 2 x 1 KB per wave
  constexpr int ASZ = BM * 256, BSZ = 128 * 128, SSZ = GS ? 1024 : 16;

  __shared__ __align__(16) char sA0[ASZ];
  __shared__ __align__(16) char sA1[ASZ];
  __shared__ __align__(16) char sA2[ASZ];
  __shared__ __align__(16) char sB0[BSZ];
  __shared__ __align__(16) char sB1[BSZ];
  __shared__ __align__(16) char sB2[BSZ];
  // group scales of the tile: the rows of k halves 0 and 1, 256 columns each
  __shared__ __align__(16) char sS0[SSZ];
  __shared__ __align__(16) char sS1[SSZ];
  __shared__ __align__(16) char sS2[SSZ];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = wave >> 2, wn0 = (wave & 3) * WN;
  int tm, tn;
  tr4_tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // split-K slice blockIdx.y covers k-tiles kt0 .. kt0 + kt_slice - 1
  const int kt0 = blockIdx.y * p.kt_slice;
  const int ktiles = p.kt_slice;
  const int last = ktiles - 1;

  // ---- DMA sources. A: instruction i of wave w fills rows 4 (4 w + i) .. +3 (lane L: row
  // L / 16, slot L % 16); B: rows 8 (2 w + i) .. +7 (lane L: row L / 8, slot L % 8). ----
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb * 4));
  int a_off[A_DMA], b_off[B_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = 4 * (A_DMA * wave + i) + (lane >> 4);
    a_off[i] = (int)((int64_t)min(m0 + r, p.M - 1) * p.lda * 2) + tr4_aslot(r, lane & 15) * 16;
  }
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) {
    const int r = 8 * (2 * wave + i) + (lane >> 3);
    b_off[i] = r * p.ql.row_bytes + tn * p.ql.tile_bytes + tr4_bslot(r, lane & 7) * 16;
  }
  // Scales: a 4-byte DMA per wave brings 128 column scales (lane L: columns 2 L, 2 L + 1) of
  // one k half's row; waves 0-3 fill both rows, waves 4-7 write the same bytes again, so every
  // wave issues the same loads.
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(p.scales, GS ? (uint32_t)((int64_t)(p.K / p.group) * p.N * 2) : 16u);
  const int s_half = (wave >> 1) & 1, s_part = wave & 1;
  const int s_off = (n0 + 128 * s_part + 2 * lane) * 2;
  auto issue = [&](int kt, char* sA, char* sB, char* sS) {
    const int k0 = (kt0 + kt) * 128;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) tr4_dma16(ra, sA + (A_DMA * wave + i) * 1024, a_off[i], k0 * 2);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) tr4_dma16(rb, sB + (2 * wave + i) * 1024, b_off[i], qrow_off(p.ql, k0));
    if constexpr (GS)
      tr4_dma4(rs, sS + 512 * s_half + 256 * s_part, s_off, ((k0 + 64 * s_half) / p.group) * p.N * 2);
  };

  // ---- fragment addresses ----
  const int l32 = lane & 31, lh = lane >> 5;
  // A: k-step s of this wave's half, fragment i: row 32 i + l32, chunk 8 h + 2 s + lh.
  // The slot XOR uses r & 15 = l32 & 15 for every fragment, so fragment i adds 32 * 256 i.
  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = l32 * 256 + (tr4_aslot(l32, 8 * h + 2 * s + lh) << 4);
  // B: fragment j, k-step pair p2 (steps 2 p2, 2 p2 + 1)
  const int g = lane >> 4, q = lane & 15;
  int boff[FN][2];
#pragma unroll
  for (int p2 = 0; p2 < 2; ++p2) {
    const int pe = q & 7;
    const int row = 64 * h + 16 * (2 * p2 + (q >> 3)) + 8 * (g >> 1) + (2 * (pe & 3) + (pe >> 2));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int seg = (wn0 + 32 * j) / 16 + (g & 1);  // 8-byte segment of 16 columns
      boff[j][p2] = row * 128 + (tr4_bslot(row, seg >> 1) << 4) + 8 * (seg & 1);
    }
  }
  // scales: column wn0 + 32 j + l32 of this wave's half
  const int s_rd = 512 * h + 2 * (wn0 + l32);

  const pk_half2 c1032 = {(pk_half)1032.0f, (pk_half)1032.0f};
  const pk_half2 c72 = {(pk_half)72.0f, (pk_half)72.0f};
  // Codes of one k-step of one fragment (raw: 8 nibbles in the tr_b4 order) times the scale
  // pair s2.
  auto dequant = [&](uint32_t raw, uint32_t s2) -> pk_half8 {
    const uint32_t d8 = raw >> 8;
    pk_half2 q0 = tr4_h2((raw & 0x000f000fu) ^ 0x64086408u) - c1032;
    pk_half2 q1 = tr4_h2((raw & 0x00f000f0u) ^ 0x54805480u) - c72;
    pk_half2 q2 = tr4_h2((d8 & 0x000f000fu) ^ 0x64086408u) - c1032;
    pk_half2 q3 = tr4_h2((d8 & 0x00f000f0u) ^ 0x54805480u) - c72;
    if constexpr (GS) {
      const pk_half2 sv = tr4_h2(s2);
      q0 = q0 * sv;
      q1 = q1 * sv;
      q2 = q2 * sv;
      q3 = q3 * sv;
    }
    return (pk_half8){q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
  };

  pk_f16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f16v){};
  pk_half8 af[2][FM];  // by k-step parity
  pk_half8 bq[2][FN];
  pk_v2i braw[2][FN][2];  // [tile parity][fragment][step pair]
  uint32_t sc[2][FN];

  auto read_a = [&](const char* sA, int s) {
#pragma unroll
    for (int i = 0; i < FM; ++i) af[s & 1][i] = *reinterpret_cast<const pk_half8*>(sA + aoff[s] + 8192 * i);
  };
  auto read_codes = [&](const char* sB, const char* sS, int par) {
#pragma unroll
    for (int p2 = 0; p2 < 2; ++p2)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        braw[par][j][p2] = __builtin_amdgcn_ds_read_tr4_b64_v2i32((__attribute__((address_space(3))) pk_v2i*)(sB + boff[j][p2]));
    if constexpr (GS) {
#pragma unroll
      for (int j = 0; j < FN; ++j) sc[par][j] = *reinterpret_cast<const uint16_t*>(sS + s_rd + 64 * j);
    }
  };
  auto pack_scales = [&](int par) {
    if constexpr (GS) {
#pragma unroll
      for (int j = 0; j < FN; ++j) sc[par][j] = sc[par][j] | (sc[par][j] << 16);
    }
  };
  auto dequant_step = [&](int s, int par) {
#pragma unroll
    for (int j = 0; j < FN; ++j) bq[s & 1][j] = dequant((uint32_t)braw[par][j][s >> 1][s & 1], sc[par][j]);
  };
  auto mfma_step = [&](int s) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bq[s & 1][j], af[s & 1][i], acc[i][j], 0, 0, 0);
  };
  auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
  // one MFMA, then up to four VALU (a 32-cycle MFMA hides them); ND DS reads early in the step
  auto pattern = [](auto ND, auto NV) {
    constexpr int nd = decltype(ND)::value, nv = decltype(NV)::value;
#pragma unroll
    for (int m = 0; m < FM * FN; ++m) {
      // DMAs one per MFMA: issued in a burst by all waves they fill the TA address FIFO
      if (m < nv) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (m < nd) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (m == FM * FN - 1 && nd > FM * FN) __builtin_amdgcn_sched_group_barrier(0x100, nd - FM * FN + 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
  };

  // DMA instructions each wave issues per tile (A, B and the scale row).
  constexpr int VPT = A_DMA + B_DMA + (GS ? 1 : 0);

  // ---- prologue: tiles 0 and 1 in flight; tile 0's codes and k-step-0 operands ready ----
  issue(0, sA0, sB0, sS0);
  issue(min(1, last), sA1, sB1, sS1);
  __builtin_amdgcn_s_waitcnt(tr4_wait_vm(VPT));
  asm volatile("s_barrier" ::: "memory");
  read_codes(sB0, sS0, 0);
  read_a(sA0, 0);
  pack_scales(0);
  dequant_step(0, 0);

  // One k-tile t (stage c; tile t+1 in stage n; stage x held tile t-1; parity par = t % 2).
  // Its k-step 0 operands are ready on entry. Steps 0 and 1 run; then every wave waits for
  // its DMA of tile t+1 and the workgroup meets (tile t+1 is in LDS, tile t-1 finished
  // everywhere), the DMA of tile t+2 goes into stage x, and steps 2 and 3 run while tile
  // t+1's codes, scales and k-step-0 A fragments are read and its k-step 0 dequantised, so the
  // next tile starts with its operands in registers. (After the last tile these reads touch
  // a stage that holds a repeat of an earlier tile and their results are not used.)
  auto tile = [&](int kt, char* sAc, char* sAn, char* sBn, char* sSn, char* sAx, char* sBx,
                  char* sSx, auto PAR) {
    constexpr int par = decltype(PAR)::value;
    fence();
    mfma_step(0);
    read_a(sAc, 1);
    dequant_step(1, par);
    pattern(pk_int_c<FM>{}, pk_int_c<0>{});
    fence();
    mfma_step(1);
    read_a(sAc, 2);
    dequant_step(2, par);
    pattern(pk_int_c<FM>{}, pk_int_c<0>{});
    fence();
    __builtin_amdgcn_s_waitcnt(tr4_wait_vm(0));
    asm volatile("s_barrier" ::: "memory");
    fence();
    issue(min(kt + 2, last), sAx, sBx, sSx);
    mfma_step(2);
    read_a(sAc, 3);
    dequant_step(3, par);
    read_codes(sBn, sSn, par ^ 1);
    pattern(pk_int_c<FM + 2 * FN + (GS ? FN : 0)>{}, pk_int_c<VPT>{});
    fence();
    mfma_step(3);
    read_a(sAn, 0);
    pack_scales(par ^ 1);
    dequant_step(0, par ^ 1);
    pattern(pk_int_c<FM>{}, pk_int_c<0>{});
    fence();
  };

  int kt = 0;
  for (; kt + 6 <= ktiles; kt += 6) {
    tile(kt, sA0, sA1, sB1, sS1, sA2, sB2, sS2, pk_int_c<0>{});
    tile(kt + 1, sA1, sA2, sB2, sS2, sA0, sB0, sS0, pk_int_c<1>{});
    tile(kt + 2, sA2, sA0, sB0, sS0, sA1, sB1, sS1, pk_int_c<0>{});
    tile(kt + 3, sA0, sA1, sB1, sS1, sA2, sB2, sS2, pk_int_c<1>{});
    tile(kt + 4, sA1, sA2, sB2, sS2, sA0, sB0, sS0, pk_int_c<0>{});
    tile(kt + 5, sA2, sA0, sB0, sS0, sA1, sB1, sS1, pk_int_c<1>{});
  }
  const int rem = ktiles - kt;
  if (rem > 0) tile(kt, sA0, sA1, sB1, sS1, sA2, sB2, sS2, pk_int_c<0>{});
  if (rem > 1) tile(kt + 1, sA1, sA2, sB2, sS2, sA0, sB0, sS0, pk_int_c<1>{});
  if (rem > 2) tile(kt + 2, sA2, sA0, sB0, sS0, sA1, sB1, sS1, pk_int_c<0>{});
  if (rem > 3) tile(kt + 3, sA0, sA1, sB1, sS1, sA2, sB2, sS2, pk_int_c<1>{});
  if (rem > 4) tile(kt + 4, sA1, sA2, sB2, sS2, sA0, sB0, sS0, pk_int_c<0>{});
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA into LDS outlives the waves
  mfma_drain();

  // ---- epilogue ----
  __syncthreads();  // every wave's last LDS reads are done: the stages are free
  // The k-half-1 waves park their accumulators in LDS, the k-half-0 waves add them: rounds of
  // four fragments (16 KB per wave, lane-major per register so each lane reads back its own
  // values; two rounds with 128-row tiles, one with 64), column wave c in its own 16 KB of stage
  // memory, which it then reuses to stage its output slices.
  const int cw = wave & 3;
  char* region;
  if constexpr (BM == 128) region = (cw < 2 ? sA0 : sA1) + (cw & 1) * 16384;
  else region = cw == 0 ? sA0 : cw == 1 ? sA1 : cw == 2 ? sA2 : sB0;
  float* const park = reinterpret_cast<float*>(region);
#pragma unroll
  for (int half = 0; half < FM / 2; ++half) {
    if (h == 1) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) park[(f * 16 + r) * 64 + lane] = acc[2 * half + f / 2][f % 2][r];
    }
    __syncthreads();
    if (h == 0) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[2 * half + f / 2][f % 2][r] += park[(f * 16 + r) * 64 + lane];
    }
    __syncthreads();
  }
  if (h == 1) return;
  // slices of the wave's 128 x 64 block staged in 8 KB (rows of 64 values, 16-byte chunks
  // XOR-swizzled by row), stored row-contiguous
  char* const stg = region;
  char* const out_base = reinterpret_cast<char*>(p.c);
  const int64_t out_off = (int64_t)blockIdx.y * p.c_slice;
  with_dtype(p.c_dtype, [&](auto DT) {
    constexpr int dt = decltype(DT)::value;
    constexpr int E = dt == PK_F32 ? 4 : 2;
    constexpr int RB = WN * E, NCH = RB / 16;  // bytes and 16-byte chunks per staged row
    constexpr int ROWS = 8192 / RB;            // rows per staged slice (32 for fp32, 64 for 16-bit)
    constexpr int FPS = ROWS / 32;             // row fragments per slice
#pragma unroll
    for (int i0 = 0; i0 < FM; i0 += FPS) {
#pragma unroll
      for (int ii = 0; ii < FPS; ++ii)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            const int r = 32 * ii + l32, col = 32 * j + 8 * qq + 4 * lh;
            const int byte = col * E;
            char* dst = stg + r * RB + ((((byte >> 4) ^ (r % NCH)) << 4) | (byte & 15));
            const pk_f4 v = p.epi((pk_f4){acc[i0 + ii][j][4 * qq], acc[i0 + ii][j][4 * qq + 1],
                                          acc[i0 + ii][j][4 * qq + 2], acc[i0 + ii][j][4 * qq + 3]},
                                  n0 + wn0 + col);
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
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the slice is in LDS
#pragma unroll
      for (int c0 = 0; c0 < ROWS * NCH; c0 += 64) {
        const int idx = c0 + lane, r = idx / NCH, ch = idx % NCH;
        const pk_u4v val = *reinterpret_cast<const pk_u4v*>(stg + r * RB + ((ch ^ (r % NCH)) << 4));
        const int gm = m0 + 32 * i0 + r, gn = n0 + wn0 + ch * (16 / E);
        // non-temporal: the output is written once and not read here (measured on MI355X:
        // 2048 x 4096 x 4096 about 4% faster than with ordinary stores)
        if (gm < p.M) __builtin_nontemporal_store(val, PK_GLOBAL(pk_u4v, out_base + (out_off + (int64_t)gm * p.ldc + gn) * E));
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // the slice is read back before the next one lands
    }
  });
}

// Shapes the kernel takes (any M: rows past M are clamped for loading and never stored).
bool tr4_shape_ok(int M, int N, int K, int group, bool has_gs) {
  if (M < 1 || N % 256 || K % 128 || K < 128) return false;
  if (has_gs && group % 64) return false;
  return true;
}

bool tr4_split_ok(int K, int split) { return split >= 1 && K % (128 * split) == 0; }

// Cost in microseconds of a tile height and split, fitted to MI355X measurements (Llama-3-8B
// layers at M = 128 .. 1024, graphs of back-to-back calls): a workgroup's k-tile of 128 takes
// about 1.23 us with 128-row tiles and 0.77 us with 64-row ones (half the MFMAs, but each int4
// fragment dequantised for half the rows and twice the weight reads per FLOP), workgroups
// beyond the 256 CUs run in further rounds, and split-K adds about 3 us plus 0.5 us per MB of
// fp32 partial planes, 1 us more for a slice count the reduce has no unrolled form for.
static double tr4_cost_us(int bm, int s, int M, int N, int K) {
  const int64_t wgs = cdiv(M, bm) * (int64_t)(N / 256) * s;
  const double rounds = (double)cdiv(wgs, 256);
  const double kt = (double)(K / 128 / s);
  double us = rounds * kt * (bm == 64 ? 0.77 : 1.23);
  if (s > 1) us += 3.0 + 0.5 * ((double)s * M * N * 4 / 1e6) + ((s & (s - 1)) ? 1.0 : 0.0);
  return us;
}

// Split for a tile height (see tr4_pick_split).
static int tr4_split_for(int bm, int M, int N, int K) {
  const int kt = K / 128;
  const int64_t tiles = cdiv(M, bm) * (int64_t)(N / 256);
  if (bm == 64) {
    // 64-row tiles: the cheapest k-split filling at most the 256 CUs by the cost model
    // (measured at M = 128: 14336 x 4096 8 slices 25.9 us, 7 27.1, 14 35.2; 4096 x 4096 4
    // slices 16.5, 8 18.4; 4096 x 6144 4 slices 19.2, 8 23.6)
    int best = 1;
    for (int s = 2; s <= 16 && s <= kt; ++s)
      if (kt % s == 0 && tiles * s <= 256 && tr4_cost_us(64, s, M, N, K) < tr4_cost_us(64, best, M, N, K))
        best = s;
    return best;
  }
  int best = 1, best_pow2 = 1;
  for (int s = 2; s <= 16 && s <= kt; ++s)
    if (kt % s == 0 && tiles * s <= 224) {
      best = s;
      if ((s & (s - 1)) == 0) best_pow2 = s;
    }
  return 2 * best_pow2 >= best ? best_pow2 : best;
}

// Tile height, 64 or 128 rows, whichever the cost model prices lower at its split. 64-row
// tiles win where they replace split-K slices by tiles: 4096 x 6144 at M = 128 22.3 -> 18.2
// us, 4096 x 14336 33.5 -> 27.7, 14336 x 4096 32.1 -> 29.2; at M = 192 every layer 6-24%;
// 128-row ones where the 64-row tiles would add rounds or double a workgroup's k-range at the
// same count (14336 x 4096 at M = 256: 45.8 against 50.6 us).
int tr4_pick_bm(int M, int N, int K) {
  return tr4_cost_us(64, tr4_split_for(64, M, N, K), M, N, K) <
                 tr4_cost_us(128, tr4_split_for(128, M, N, K), M, N, K)
             ? 64
             : 128;
}

// Split-K for the shape: the most equal k-slices (a divisor of K / 128, at most 16) that keep
// tiles x slices <= 224 workgroups, one slice wherever that is 1. Measured on MI355X (M = 65 to
// 1024 at K = 4096 and 14336, N = 4096 to 14336): each slice costs its fp32 partial plane
// written and read back plus the reduce launch (about 7 us of fixed cost and 0.34 us per MB of
// planes), while k-tile time rises from 1.4 us with up to 128 busy CUs to 1.9 us with all 256,
// so the best split stops short of filling every CU.
// With 128-row tiles the most slices (dividing the k-tiles, at most 16, tiles x slices <= 224
// workgroups), but a power of two when one reaches at least half of that: fewer fp32 partial
// planes for the reduce to read, and its unrolled form. Measured on MI355X with 128-row tiles
// at M = 128, 14336 x 4096 (graphs over 22 rotating block-layout copies, GEMM + reduce): 14
// slices 36.1 us, 8 slices 32.0, 7 slices 35.5, 16 slices 37.1; 4096 x 6144: 8 slices 21.5, 4
// 22.5.
int tr4_pick_split(int M, int N, int K) { return tr4_split_for(tr4_pick_bm(M, N, K), M, N, K); }

bool tr4_ok(int M, int N, int K, int group, bool has_gs, int64_t lda, const void* b, int64_t ldb,
            int64_t ldc, int c_dtype, const void* c, int split) {
  if (!tr4_shape_ok(M, N, K, group, has_gs) || !tr4_split_ok(K, split)) return false;
  if (lda % 8) return false;
  // B is DMA'd in 16-byte chunks at k * ldb * 4 + 16 * j: 16-byte aligned base and rows
  if ((reinterpret_cast<uintptr_t>(b) & 15) || ldb % 4) return false;
  // unsplit: the epilogue stores 16-byte chunks of the output itself
  const int esz = c_dtype == PK_F32 ? 4 : 2;
  if (split == 1 && ((ldc * esz) % 16 || (reinterpret_cast<uintptr_t>(c) & 15))) return false;
  // 32-bit buffer offsets
  if ((int64_t)M * lda * 2 >= (1ll << 31)) return false;
  if ((int64_t)K * ldb * 4 >= (1ll << 31)) return false;
  return true;
}

// split > 1: slice s writes its fp32 partial plane s of the workspace (one full k-range
// product per (tile, slice)), then the fixed-order reduce adds the planes and applies the
// tensor scale (partials_only: the planes alone, at `workspace` itself).
int tr4_launch(const void* a, int64_t lda, const void* b, int64_t ldb, const void* scales,
               int group, OutEpi epi, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
               int split, void* workspace, hipStream_t s, bool partials_only, bool tiled) {
  Tr4Params p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.b = reinterpret_cast<const uint32_t*>(b);
  p.ldb = ldb;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = group > 0 ? group : K;
  p.M = M;
  p.N = N;
  p.K = K;
  const int bm = tr4_pick_bm(M, N, K);
  p.tiles_m = (int)cdiv(M, bm);
  p.tiles_n = N / 256;
  p.kt_slice = K / 128 / split;
  p.ql = qlayout(tiled, ldb, N);
  float* const partials = split > 1 ? split_partials(workspace, partials_only) : nullptr;
  if (split > 1) {
    p.epi = OutEpi(1.0f);
    p.c = partials;
    p.c_dtype = PK_F32;
    p.ldc = N;
    p.c_slice = (int64_t)M * N;
  } else {
    p.epi = epi;
    p.c = c;
    p.c_dtype = c_dtype;
    p.ldc = ldc;
    p.c_slice = 0;
  }
  const dim3 grid(p.tiles_m * p.tiles_n, split);
  if (bm == 64) {
    if (scales) w4a16_tr4_kernel<true, 64><<<grid, 512, 0, s>>>(p);
    else w4a16_tr4_kernel<false, 64><<<grid, 512, 0, s>>>(p);
  } else {
    if (scales) w4a16_tr4_kernel<true, 128><<<grid, 512, 0, s>>>(p);
    else w4a16_tr4_kernel<false, 128><<<grid, 512, 0, s>>>(p);
  }
  PK_LAUNCH_CHECK("w4a16 gemm (int4 B in LDS)");
  if (split <= 1 || partials_only) return PK_OK;
  return splitk_reduce(partials, split, M, N, epi, c, c_dtype, ldc, s);
}

}  // namespace pk
