// e4m3 fp8 GEMM for gfx950, 256 x 256 (or 256 x 128) tiles, LDS pipeline of four B stages
// and three A buffers of two k-tiles, both operands through LDS DMA
// (v_mfma_f32_32x32x64_f8f6f4).
//
// C[m, n] = out_scale * sum_k A[m, k] * B[k, n] (gemm_fp8.py:38-117), A (M, K) row-major,
// B (K, N) row-major (BLAYOUT 0) or (N, K) row-major (BLAYOUT 1, a transposed view).
//
// Design:
//  * 8 waves (2 x 4), each a 128 x 64 block: 4 x 2 fragments of 32 x 32, 64 k per MFMA.
//    256 x 128 tiles (for outputs whose 256 x 256 tiles would leave CUs idle: 2048 x 4096
//    is 128 of them for 256 CUs) use 4 x 2 waves of 64 x 64 (2 x 2 fragments), a B stage of
//    8 KB and one B DMA per wave and tile.
//  * K tiles of 64. B tile = 64 k x 256 n (BLAYOUT 0) or 256 n x 64 k (BLAYOUT 1) per stage;
//    A goes in pairs of k-tiles, 256 rows x 128 bytes per buffer, so every A DMA reads whole
//    128-byte lines (one k-tile per DMA read half lines: measured on MI355X, 4096^3 +2.3%,
//    2048 x 4096 x 4096 +6% with pairs). Both go global -> LDS with buffer DMA (no VGPR
//    staging).
//  * Four B stages and three A pair buffers (160 KB at 256 x 256). One barrier per tile, in
//    its middle: each tile's first half of MFMAs runs on fragments read during the previous
//    tile, the barrier publishes tile t+1 (whose DMAs went out two or more tiles earlier), the
//    DMAs of B tile t+3 go into tile t-1's stage and, at even t, those of A pair t/2 + 2 into
//    the buffer of tiles t-2 and t-1, and the second half of MFMAs runs while tile t+1's
//    fragments are read into registers -- no wave waits on LDS reads after the barrier.
//  * LDS rows: A's 128-byte rows in 8 chunks of 16 B, chunk c of row r in slot
//    c ^ ((r >> 1) & 7); B^T's 64-byte rows in 4 chunks, chunk c of row r in slot
//    c ^ ((r >> 2) & 3): 16 lanes reading 16 consecutive rows at one chunk hit 16 distinct
//    16-byte bank groups.
//  * (K, N) B keeps n contiguous (256-byte rows, 16 chunks, chunk c of row k in slot
//    c ^ 2(k & 7)) and is read with ds_read_b64_tr_b8: within a 16-lane group lane j gets
//    byte b from the address of lane 2b + j/8 at offset j % 8. Even lanes address row k0 + b
//    at column n, odd lanes the same row at column n + 8, so lane j receives 8 consecutive
//    k of column n + j -- the MFMA operand layout -- with no transposing in registers.
//  * The MFMAs take B as the first operand, so each accumulator is C^T and every lane ends
//    with four consecutive columns of one row per register quad. Stored directly, one store
//    instruction would write 8 or 16 bytes into each of 32 rows; instead each wave stages its
//    block through free LDS (a half pair buffer or a B stage) and writes whole 128-byte lines
//    (measured on MI355X: the 4096^3 fp16-output GEMM 10% faster).
#include "pk_internal.h"

namespace pk {

#define PK_LDS(p) ((__attribute__((address_space(3))) void*)(p))

typedef int pk_i2v __attribute__((ext_vector_type(2)));

struct F8Params {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  float scale;
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
};

// 16 bytes per lane, global -> LDS (lane L writes lds + 16 L).
__device__ __forceinline__ void f8_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS(lds), 16, voff, soff, 0, 0);
}

__device__ __forceinline__ pk_i2v f8_read_tr(const char* lds) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) pk_i2v*)(lds));
}

// slot of chunk c of row r in a 64-byte-row tile
__device__ __forceinline__ int f8_swz64(int r, int c) { return (r << 6) + ((c ^ ((r >> 2) & 3)) << 4); }
// slot of chunk c of row k in a 256-byte-row tile
__device__ __forceinline__ int f8_swz256(int k, int c) { return (k << 8) + ((c ^ (2 * (k & 7))) << 4); }
// slot of chunk c of row k in a 128-byte-row tile: the 8 rows a transposing read touches at
// one chunk land in 8 distinct 16-byte bank groups
__device__ __forceinline__ int f8_swz128(int k, int c) { return (k << 7) + ((c ^ (k & 7)) << 4); }
template <int BN>
__device__ __forceinline__ int f8_swzB(int k, int c) { return BN == 256 ? f8_swz256(k, c) : f8_swz128(k, c); }

// XCD-aware tile order: consecutive logical tiles on one XCD, grouped GROUP_M tile rows deep
// (measured on MI355X: 256 x 256 tiles at 4096^3 best at 4 rows, 2 within 0.3%, 8 and 16
// 1-2% slower; the 256 x 128 tiles of 2048 x 4096 x 4096 2.2% faster at 2 rows than at 4).
template <int GROUP_M>
__device__ __forceinline__ void f8_tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int total = tiles_m * tiles_n;
  int logical = bid;
  if (total % 8 == 0) logical = (bid % 8) * (total / 8) + bid / 8;
  const int per_group = GROUP_M * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_g = logical - g * per_group;
  *tm = first_m + in_g % gm;
  *tn = in_g / gm;
}

template <int I, int N, class F>
__device__ __forceinline__ void f8_static_for(F&& f) {
  if constexpr (I < N) {
    f(pk_int_c<I>{});
    f8_static_for<I + 1, N>(f);
  }
}

template <int BLAYOUT, int BN>
__global__ __launch_bounds__(512) void gemm_f8_v3_kernel(F8Params p) {
  constexpr int BM = 256, BK = 64;
  constexpr int WAVES_N = BN / 64, WAVES_M = 8 / WAVES_N;
  constexpr int WTM = BM / WAVES_M, WTN = 64, FM = WTM / 32, FN = 2;
  constexpr int APAIR = 2 * BM * BK;  // bytes of A per pair of k-tiles (32 KB): 128-byte rows
  constexpr int STAGE_B = BN * BK;    // bytes of B per stage
  constexpr int NBD = BN / 128;       // B DMA instructions per wave and tile
  constexpr int NAD = APAIR / 8192;   // A DMA instructions per wave and pair of k-tiles (4)

  // A in three buffers of a k-tile pair each (every DMA reads whole 128-byte lines: a row's
  // 128 k-bytes of two k-tiles), B in four stages of one k-tile.
  __shared__ __align__(16) char sAP0[APAIR];
  __shared__ __align__(16) char sAP1[APAIR];
  __shared__ __align__(16) char sAP2[APAIR];
  __shared__ __align__(16) char sB0[STAGE_B];
  __shared__ __align__(16) char sB1[STAGE_B];
  __shared__ __align__(16) char sB2[STAGE_B];
  __shared__ __align__(16) char sB3[STAGE_B];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm0 = (wave / WAVES_N) * WTM, wn0 = (wave % WAVES_N) * WTN;
  int tm, tn;
  f8_tile_of<BN == 128 ? 2 : 4>(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  // The last row of tiles ends at row M (M >= BM): where M % BM != 0 it overlaps the row of
  // tiles before it, whose rows it computes to the same bits, so no A row past M is read.
  const int m0 = min(tm * BM, p.M - BM), n0 = tn * BN;
  const int ktiles = p.K / BK;

  // ---- DMA sources. A: NAD = 4 1 KB instructions per wave and k-tile pair, instruction i
  // rows (4 wave + i) * 8 .. +7 of 128 bytes (lane L: row + L / 8, slot L % 8 holding chunk
  // (L % 8) ^ ((row >> 1) & 7)); instructions 2 and 3 are 0 and 1 sixteen rows on (the same
  // chunk pattern), by the scalar offset. Every row read is < M (the tile row above) and
  // every k < K (K % 128 == 0: whole pairs), so no access depends on how the hardware
  // range-checks the scalar offset. B: NBD per wave and k-tile ----
  static_assert(NAD == 4, "four A instructions per wave and pair");
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda));
  int a_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * NAD + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_off[i] = (int)((int64_t)(m0 + r) * p.lda) + c * 16;
  }
  const int a_skip = 16 * (int)p.lda;  // bytes of 16 rows
  __amdgpu_buffer_rsrc_t rb;
  int b_off[NBD];
  if constexpr (BLAYOUT == 1) {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.N * p.ldb));
#pragma unroll
    for (int i = 0; i < NBD; ++i) {
      const int r = (wave * NBD + i) * 16 + (lane >> 2);
      const int c = (lane & 3) ^ ((r >> 2) & 3);
      b_off[i] = (int)((int64_t)min(n0 + r, p.N - 1) * p.ldb) + c * 16;
    }
  } else {
    rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb));
    constexpr int CPR = BN / 16;  // 16-byte chunks per k row
#pragma unroll
    for (int i = 0; i < NBD; ++i) {
      const int k = (wave * NBD + i) * (64 / CPR) + lane / CPR;  // 1 KB of k rows per instruction
      const int c = BN == 256 ? (lane & 15) ^ (2 * (k & 7)) : (lane & 7) ^ (k & 7);
      b_off[i] = (int)((int64_t)k * p.ldb) + min(n0 + c * 16, p.N - 16);
    }
  }
  // B of k-tile kt; A of k-tile pair kp (k-tiles 2 kp, 2 kp + 1).
  auto issue_b = [&](int kt, char* sB) {
    const int bs = BLAYOUT == 1 ? kt * BK : (int)((int64_t)kt * BK * p.ldb);
#pragma unroll
    for (int i = 0; i < NBD; ++i) f8_dma16(rb, sB + (wave * NBD + i) * 1024, b_off[i], bs);
  };
  auto issue_a = [&](int kp, char* sAP) {
#pragma unroll
    for (int i = 0; i < NAD; ++i)
      f8_dma16(ra, sAP + (wave * NAD + i) * 1024, a_off[i & 1], kp * 2 * BK + (i >> 1) * a_skip);
  };

  // ---- fragment offsets. A, in a pair buffer: row r, 16-byte chunk c of k-tile half hf at
  // slot (4 hf + c) ^ ((r >> 1) & 7) -- the second half's offset is the first's XOR 64. The 16
  // rows a 16-lane group reads at one chunk cover all 16 bank groups. ----
  // Fragment row i adds 32 * 128 bytes (the swizzle depends on (lane & 31) only, wm0 and 32 i
  // being multiples of 32), so one register per (half, chunk) covers every fragment row.
  int aoff[2][2];  // [k-tile half][chunk of the lane's pair]
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = wm0 + (lane & 31), c = 4 * hf + 2 * (lane >> 5) + h;
      aoff[hf][h] = r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
    }
  // BLAYOUT 1: [j][h] chunk pair, fragment j adding 32 rows of 64 bytes to j = 0's (the swizzle
  // depends on (lane & 31) only); BLAYOUT 0: [j][0] transposing reads, read q adding 8 k rows
  // (the swizzle depends on k & 7 only).
  int boff[FN][2];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if constexpr (BLAYOUT == 1) {
#pragma unroll
      for (int h = 0; h < 2; ++h) boff[j][h] = f8_swz64(wn0 + (lane & 31), 2 * (lane >> 5) + h);
    } else {
      const int i16 = lane & 15;
      const int cs = wn0 + 32 * j + 16 * ((lane >> 4) & 1) + 8 * (i16 & 1);  // first column
      const int k = 32 * (lane >> 5) + (i16 >> 1);
      boff[j][0] = f8_swzB<BN>(k, cs >> 4) + (cs & 15);
      boff[j][1] = 0;
    }
  }

  pk_f16v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (pk_f16v){};

  // Operand registers: A fragments (the first part's are reloaded for the next tile while the
  // second part runs) and B fragments by tile parity. The first part is P1 fragment rows.
  constexpr int HF = FM / 2;
  constexpr int P1 = HF;
  pk_i8v af[FM];
  pk_i8v bf[2][FN];
  auto read_b = [&](const char* sB, int par) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (BLAYOUT == 1) {
        const pk_u4v x0 = *reinterpret_cast<const pk_u4v*>(sB + boff[0][0] + 2048 * j);
        const pk_u4v x1 = *reinterpret_cast<const pk_u4v*>(sB + boff[0][1] + 2048 * j);
        bf[par][j] = (pk_i8v){(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
      } else {
        constexpr int KQ = 8 * BN;  // bytes of 8 k rows
        const pk_i2v y0 = f8_read_tr(sB + boff[j][0]);
        const pk_i2v y1 = f8_read_tr(sB + boff[j][0] + KQ);
        const pk_i2v y2 = f8_read_tr(sB + boff[j][0] + 2 * KQ);
        const pk_i2v y3 = f8_read_tr(sB + boff[j][0] + 3 * KQ);
        bf[par][j] = (pk_i8v){y0[0], y0[1], y1[0], y1[1], y2[0], y2[1], y3[0], y3[1]};
      }
    }
  };
  auto read_a = [&](const char* sAP, int hf, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      const pk_u4v x0 = *reinterpret_cast<const pk_u4v*>(sAP + aoff[hf][0] + 4096 * i);
      const pk_u4v x1 = *reinterpret_cast<const pk_u4v*>(sAP + aoff[hf][1] + 4096 * i);
      af[i] = (pk_i8v){(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
    }
  };
  auto mfma_rows = [&](int i0, int i1, int par) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[par][j], af[i], acc[i][j], 0, 0, 0, 0, 0, 0);
  };
  auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
  // NM MFMAs with ND LDS reads and NV DMAs spread between them.
  auto pattern = [](auto NM, auto ND, auto NV) {
    constexpr int nd = decltype(ND)::value, nv = decltype(NV)::value;
    constexpr int nm = decltype(NM)::value;
    constexpr int dper = (nd + nm - 1) / nm;
#pragma unroll
    for (int m = 0; m < nm; ++m) {
      if (m < nv) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (m * dper < nd) __builtin_amdgcn_sched_group_barrier(0x100, dper, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  };

  // ---- pipeline. Tile t (B stage t % 4, A pair buffer (t / 2) % 3, half t % 2) starts with
  // its B fragments and first-half A fragments in registers. First half: MFMAs of rows
  // 0 .. HF-1 while the second half's A fragments are read. Then every wave waits for its DMAs
  // of tile t+1 and the workgroup meets (tile t+1 is in LDS everywhere; every wave has
  // finished tile t-1, so its B stage is free, and at even t so is the pair buffer of tiles
  // t-2 and t-1), and the DMAs of B tile t+3 and, at even t, of A pair t/2 + 2 (tiles t+4 and
  // t+5) go into those, between the second half's MFMAs, which also read tile t+1's B and
  // first-half A fragments: the next tile starts with its operands in registers and no wave
  // waits on LDS after the barrier. Tiles past the end are re-reads of the last tile (pair)
  // into a stage nobody reads, so the DMA count in flight is the same at every barrier: after
  // B tile t+1 come B tile t+2 and one A pair, NBD + NAD instructions.
  const int last = ktiles - 1, lastp = last / 2;
  issue_a(0, sAP0);
  issue_b(0, sB0);
  issue_b(min(1, last), sB1);
  issue_a(min(1, lastp), sAP1);
  issue_b(min(2, last), sB2);
  // s_waitcnt vmcnt(n) expcnt(7) lgkmcnt(15). The barrier is a bare s_barrier: __syncthreads()
  // adds a workgroup release fence, which waits for *every* outstanding LDS DMA (vmcnt(0)) and
  // would serialise the pipeline. The explicit wait covers the data the barrier publishes, and
  // the asm memory clobber keeps the compiler from moving LDS accesses across it.
  constexpr int kWaitTile0 = 0x0f70 | (2 * NBD + NAD);  // A pair 0 and B tile 0 landed
  constexpr int kWaitNext = 0x0f70 | (NBD + NAD);       // B tile t+1 (and A of t+1) landed
  static_assert(2 * NBD + NAD < 16, "vmcnt fits the immediate's low field");
  __builtin_amdgcn_s_waitcnt(kWaitTile0);
  asm volatile("s_barrier" ::: "memory");
  read_b(sB0, 0);
  read_a(sAP0, 0, 0, P1);

  auto step = [&](int kt, const char* sAPc, const char* sAPn, const char* sBn, char* sBx,
                  char* sAPx, auto U) {
    constexpr int u = decltype(U)::value;
    constexpr int par = u & 1, hc = u & 1, hn = (u + 1) & 1;
    constexpr bool issue_pair = (u & 1) == 0;
    fence();
    mfma_rows(0, P1, par);
    read_a(sAPc, hc, P1, FM);
    pattern(pk_int_c<P1 * FN>{}, pk_int_c<2 * (FM - P1)>{}, pk_int_c<0>{});
    fence();
    __builtin_amdgcn_s_waitcnt(kWaitNext);
    asm volatile("s_barrier" ::: "memory");
    fence();
    issue_b(min(kt + 3, last), sBx);
    if constexpr (issue_pair) issue_a(min(kt / 2 + 2, lastp), sAPx);
    mfma_rows(P1, FM, par);
    read_b(sBn, par ^ 1);
    read_a(sAPn, hn, 0, P1);
    pattern(pk_int_c<(FM - P1) * FN>{}, pk_int_c<(BLAYOUT == 1 ? 2 : 4) * FN + 2 * P1>{},
            pk_int_c<NBD + (issue_pair ? NAD : 0)>{});
    fence();
  };
  // 12 tiles per pass: the B stages cycle every 4, the A pair buffers every 6.
  auto sap = [&](int i) -> char* { return i == 0 ? sAP0 : i == 1 ? sAP1 : sAP2; };
  auto sbs = [&](int i) -> char* { return i == 0 ? sB0 : i == 1 ? sB1 : i == 2 ? sB2 : sB3; };
  auto step_u = [&](int kt, auto U) {
    constexpr int u = decltype(U)::value;
    step(kt, sap((u / 2) % 3), sap(((u + 1) / 2) % 3), sbs((u + 1) % 4), sbs((u + 3) % 4),
         sap((u / 2 + 2) % 3), U);
  };
  int kt = 0;
  for (; kt + 11 < ktiles; kt += 12)
    f8_static_for<0, 12>([&](auto U) { step_u(kt + decltype(U)::value, U); });
  f8_static_for<0, 11>([&](auto U) {
    if (kt + decltype(U)::value < ktiles) step_u(kt + decltype(U)::value, U);
  });
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA into LDS outlives the waves
  mfma_drain();

  // ---- epilogue ----
  // Through LDS when rows are 16-byte aligned: each wave stages halves of its block (64 rows
  // of 128 x 64, or 32 rows of 64 x 64) in a free stage region of its own (rows of 64 values,
  // 16-byte chunks XOR-swizzled by row), then writes them back row-contiguous, 16 bytes per
  // lane: every store instruction covers whole 128-byte lines instead of 16 bytes in each of
  // 32 rows.
  const int esz = p.c_dtype == PK_F32 ? 4 : 2;
  const bool vec16 = (p.ldc * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0;
  const int em = lane & 31, en = 4 * (lane >> 5);
  if (vec16) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS reads are done
    __syncthreads();                     // and every other wave's: the stages are free
    // a wave-uniform region of 64 rows x 64 fp32 (16 KB; 256 x 128 tiles: 32 rows, 8 KB)
    char* sW;
    if constexpr (BN == 256)  // 16 KB each: halves of the pair buffers, B stages 0 and 1
      sW = wave < 2 ? sAP0 + wave * 16384 : wave < 4 ? sAP1 + (wave - 2) * 16384
         : wave < 6 ? sAP2 + (wave - 4) * 16384 : wave == 6 ? sB0 : sB1;
    else  // 8 KB each: quarters of pair buffers 0 and 1
      sW = (wave < 4 ? sAP0 : sAP1) + (wave & 3) * 8192;
    with_dtype(p.c_dtype, [&](auto DT) {
      constexpr int dt = decltype(DT)::value;
      constexpr int E = dt == PK_F32 ? 4 : 2;
      constexpr int RB = 64 * E, NCH = RB / 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < HF; ++ii)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = 32 * ii + em, col = 32 * j + 8 * q + en;
              const int byte = col * E;
              char* dst = sW + r * RB + ((((byte >> 4) ^ (r % NCH)) << 4) | (byte & 15));
              const pk_f4 acc4 = {acc[HF * h + ii][j][4 * q], acc[HF * h + ii][j][4 * q + 1],
                                  acc[HF * h + ii][j][4 * q + 2], acc[HF * h + ii][j][4 * q + 3]};
              const pk_f4 v = acc4 * p.scale;
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
        for (int c0 = 0; c0 < 32 * HF * NCH; c0 += 64) {
          const int idx = c0 + lane, r = idx / NCH, ch = idx % NCH;
          const pk_u4v val = *reinterpret_cast<const pk_u4v*>(sW + r * RB + ((ch ^ (r % NCH)) << 4));
          const int gm = m0 + wm0 + 32 * HF * h + r, gn = n0 + wn0 + ch * (16 / E);
          if (gm < p.M && gn < p.N)  // N % 16 == 0: a chunk is all in or all out
            // non-temporal: written once, read by no later part of this kernel (measured on
            // MI355X: 2048x4096x4096 2-4% faster, 4096^3 +0.5%)
            __builtin_nontemporal_store(val, PK_GLOBAL(pk_u4v, reinterpret_cast<char*>(p.c) + ((int64_t)gm * p.ldc + gn) * E));
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next half is staged
      }
    });
    return;
  }
  const bool vec = p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & (4 * esz - 1)) == 0;
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
            v *= p.scale;
            store4_as<dt>(p.c, (int64_t)gm * p.ldc + gn, v, vec);
          }
        }
  });
}

bool f8_v3_ok(int M, int N, int K, int64_t lda, int64_t ldb, int b_layout, const void* b) {
  if (M < 256 || N < 256 || K % 128 || N % 16 || lda % 16 || ldb % 16) return false;
  if ((reinterpret_cast<uintptr_t>(b) & 15) != 0) return false;
  if ((int64_t)M * lda >= (1ll << 31)) return false;
  return (b_layout == 1 ? (int64_t)N * ldb : (int64_t)K * ldb) < (1ll << 31);
}

int f8_v3_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s) {
  F8Params p;
  p.a = a8;
  p.lda = lda;
  p.b = b8;
  p.ldb = ldb;
  p.scale = out_scale;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (int)cdiv(M, 256);
  // 256 x 128 tiles where 256 x 256 ones would leave CUs idle
  int cus = 256;
  {
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
      (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  }
  const bool narrow = (int64_t)p.tiles_m * cdiv(N, 256) < cus;
  p.tiles_n = (int)cdiv(N, narrow ? 128 : 256);
  const dim3 grid(p.tiles_m * p.tiles_n);
  if (narrow) {
    if (b_layout == 1) gemm_f8_v3_kernel<1, 128><<<grid, 512, 0, s>>>(p);
    else gemm_f8_v3_kernel<0, 128><<<grid, 512, 0, s>>>(p);
  } else {
    if (b_layout == 1) gemm_f8_v3_kernel<1, 256><<<grid, 512, 0, s>>>(p);
    else gemm_f8_v3_kernel<0, 256><<<grid, 512, 0, s>>>(p);
  }
  PK_LAUNCH_CHECK("fp8 gemm (v3)");
  return PK_OK;
}

}  // namespace pk
