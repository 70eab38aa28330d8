// W4A16 GEMM for large outputs on gfx950: 256 x 256 tiles, 8 waves of 128 x 64 each,
// v_mfma_f32_16x16x32_f16, four LDS stages of 32 k (gemm_int4.py:22-107 is the operation:
// C = A @ dequant(B), B int4 codes packed 8 per int32 along N, fp16 group scales along K).
//
// Why this shape: per k-tile a wave reads (128 + 64) x 32 fp16 from LDS for 32 MFMAs, a
// quarter less LDS traffic per FLOP than 64 x 64 wave blocks; with A DMA'd and B dequantised
// into LDS the loop then needs about 130 KB of LDS traffic per 1024 matrix-pipe cycles of a
// CU, like the fp8 kernel's (gemm_f8_v3.hip).
//
// Design:
//  * A (M, K) fp16 goes global -> LDS by buffer DMA, 256 rows x 64 bytes per stage, chunk c
//    of row r in slot c ^ ((r >> 2) & 3).
//  * B: thread t owns word column t / 16 (8 output columns) and rows 2 (t % 16) + {0, 1} of
//    the k-tile. Its two words are loaded two tiles ahead, dequantised one tile ahead --
//    (q & 0xF) | 0x6400 - 1032 gives the exact code in fp16, times the fp16 group scale, the
//    arithmetic of the 256 x 128 kernel (gemm_v2.hip), so both produce the same bits -- and
//    written k-contiguous: one 4-byte (k, k+1) pair per output column into rows of 64 bytes.
//    Row n sits at position (n & ~3) | ((n + (n >> 3)) & 3) of its group of four, so the four
//    16-lane groups of a write instruction (word columns 4w .. 4w+3) land in four different
//    bank quarters, and 16 consecutive rows read at one chunk still cover all 64 banks.
//  * One barrier per k-tile. After it: the B words of tile t+2 are requested, the tile's
//    fragments read, and its 32 MFMAs issued in groups of four with the A DMA of tile t+3 and the
//    dequantisation of tile t+1 woven between them (a wave issues in order, so its VALU and
//    memory work overlap its matrix-pipe work only when placed between MFMAs).
//  * 16 x 16 x 32 MFMAs (8 x 4 per wave and k-tile): the same operand bytes and matrix-pipe
//    time per FLOP as 32 x 32 x 16, in four times as many instructions to weave the DMA and
//    dequantisation work between (measured on MI355X: 3-5% faster on large dense shapes).
//    They take B as the first operand (each accumulator is C^T): lane l holds columns
//    4 (l / 16) .. +3 of row l % 16 of its fragment; the epilogue stages each wave's block in
//    a free stage array and writes whole 128-byte lines.
#include "pk_internal.h"

namespace pk {

#define PK_LDS(p) ((__attribute__((address_space(3))) void*)(p))

struct W4WideParams {
  const pk_half* a;
  int64_t lda;            // elements
  const uint32_t* b;      // int4 words (K, N / 8)
  int64_t ldb;            // words
  const pk_half* scales;  // (K / group, N) or null
  int group;
  float scale;            // epilogue scale (tensor scale)
  void* c;
  int c_dtype;
  int64_t ldc;
  int M, N, K;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ void w4w_dma16(__amdgpu_buffer_rsrc_t r, char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, PK_LDS(lds), 16, voff, soff, 0, 0);
}

// Byte offset of chunk c (16 bytes = 8 k) of A row r in a stage.
__device__ __forceinline__ int w4w_aswz(int r, int c) { return (r << 6) + ((c ^ ((r >> 2) & 3)) << 4); }
// Byte offset of chunk c of B column n (a row of the k-contiguous B^T tile).
__device__ __forceinline__ int w4w_bswz(int n, int c) {
  const int pos = (n & ~3) | ((n + (n >> 3)) & 3);
  return (pos << 6) + ((c ^ ((n >> 2) & 3)) << 4);
}

__device__ __forceinline__ pk_half2 w4w_h2(uint32_t v) { return __builtin_bit_cast(pk_half2, v); }
__device__ __forceinline__ uint32_t w4w_u32(pk_half2 v) { return __builtin_bit_cast(uint32_t, v); }

// XCD-aware tile order: consecutive logical tiles on one XCD, grouped 4 tile rows deep.
__device__ __forceinline__ void w4w_tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
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

template <bool GS>
__global__ __launch_bounds__(512) void gemm_w4_wide_kernel(W4WideParams p) {
  constexpr int BM = 256, BK = 32;
  constexpr int WTM = 128, WTN = 64, GM = WTM / 16, GN = WTN / 16;
  constexpr int STAGE = BM * BK * 2;  // bytes per operand per stage (16 KB)

  __shared__ __align__(16) char sA0[STAGE];
  __shared__ __align__(16) char sA1[STAGE];
  __shared__ __align__(16) char sA2[STAGE];
  __shared__ __align__(16) char sA3[STAGE];
  __shared__ __align__(16) char sB0[STAGE];
  __shared__ __align__(16) char sB1[STAGE];
  __shared__ __align__(16) char sB2[STAGE];
  __shared__ __align__(16) char sB3[STAGE];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm0 = (wave >> 2) * WTM, wn0 = (wave & 3) * WTN;
  int tm, tn;
  w4w_tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int m0 = tm * BM, n0 = tn * 256;
  const int ktiles = p.K / BK;
  const int last = ktiles - 1;

  // ---- A: two 1 KB DMA instructions per wave per tile (16 rows of 64 bytes each) ----
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, (uint32_t)((int64_t)p.M * p.lda * 2));
  int a_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * 2 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    a_off[i] = (int)((int64_t)min(m0 + r, p.M - 1) * p.lda * 2) + c * 16;
  }
  auto issue_a_part = [&](int kt, char* sA, int part) {
    w4w_dma16(ra, sA + (wave * 2 + part) * 1024, a_off[part], kt * BK * 2);
  };

  // ---- B words and scales of a tile into a register slot ----
  const int kp = t & 15, wc = t >> 4;
  const int wcol = min((n0 >> 3) + wc, (p.N >> 3) - 1);  // past-the-end columns re-read the last
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, (uint32_t)((int64_t)p.K * p.ldb * 4));
  const int b_off0 = (int)(((int64_t)2 * kp * p.ldb + wcol) * 4);
  const int b_off1 = b_off0 + (int)(p.ldb * 4);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(p.scales, GS ? (uint32_t)((int64_t)(p.K / p.group) * p.N * 2) : 16u);
  uint32_t bw[2][2];
  pk_u4v bs[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  auto load_b = [&](int kt, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const int k0 = kt * BK;
    const int soff = (int)((int64_t)k0 * p.ldb * 4);
    bw[sl][0] = __builtin_amdgcn_raw_buffer_load_b32(rb, b_off0, soff, 0);
    bw[sl][1] = __builtin_amdgcn_raw_buffer_load_b32(rb, b_off1, soff, 0);
    if constexpr (GS) bs[sl] = __builtin_amdgcn_raw_buffer_load_b128(rs, wcol * 16, (k0 / p.group) * p.N * 2, 0);
  };
  // Dequantise byte b (output columns 2b, 2b+1) of the slot's two words and write both
  // (k, k+1) pairs into stage sB.
  const pk_half2 bias = {(pk_half)1032.0f, (pk_half)1032.0f};
  auto dq_put = [&](auto SLOT, char* sB, int b) {
    constexpr int sl = decltype(SLOT)::value;
    const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
    const uint32_t pr = __builtin_amdgcn_perm(bw[sl][1] ^ 0x88888888u, bw[sl][0] ^ 0x88888888u, sel);
    pk_half2 lo = w4w_h2((pr & 0x000f000fu) | 0x64006400u) - bias;  // exact codes
    pk_half2 hi = w4w_h2(((pr >> 4) & 0x000f000fu) | 0x64006400u) - bias;
    if constexpr (GS) {
      const uint32_t sv = bs[sl][b];
      const pk_half2 s2 = w4w_h2(sv);
      lo = lo * s2.xx;  // (s_lo, s_lo): an operand select of the packed multiply
      hi = hi * s2.yy;
    }
    const int n = wc * 8 + 2 * b;
    const int within = (kp & 3) * 4;
    *reinterpret_cast<uint32_t*>(sB + w4w_bswz(n, kp >> 2) + within) = w4w_u32(lo);
    *reinterpret_cast<uint32_t*>(sB + w4w_bswz(n + 1, kp >> 2) + within) = w4w_u32(hi);
  };

  // ---- fragment offsets: lane l reads k 8 (l / 16) .. +7 (chunk l / 16) of row l % 16 ----
  int aoff[GM], boff[GN];
#pragma unroll
  for (int i = 0; i < GM; ++i) aoff[i] = w4w_aswz(wm0 + 16 * i + (lane & 15), lane >> 4);
#pragma unroll
  for (int j = 0; j < GN; ++j) boff[j] = w4w_bswz(wn0 + 16 * j + (lane & 15), lane >> 4);

  pk_f4 acc[GM][GN];
#pragma unroll
  for (int i = 0; i < GM; ++i)
#pragma unroll
    for (int j = 0; j < GN; ++j) acc[i][j] = (pk_f4){0.0f, 0.0f, 0.0f, 0.0f};

  // One k-tile: fragments, then 8 groups of 4 MFMAs with A DMA parts and dequantisation
  // pieces between them.
  auto compute = [&](const char* sA, const char* sB, int kta, char* sAn, auto DSLOT, char* sBd) {
    pk_half8 af[GM], bf[GN];
#pragma unroll
    for (int j = 0; j < GN; ++j) bf[j] = *reinterpret_cast<const pk_half8*>(sB + boff[j]);
#pragma unroll
    for (int i = 0; i < GM; ++i) af[i] = *reinterpret_cast<const pk_half8*>(sA + aoff[i]);
#pragma unroll
    for (int ps = 0; ps < GM; ++ps) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < GN; ++j)
        acc[ps][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[ps], acc[ps][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (ps == 0 || ps == 2) issue_a_part(kta, sAn, ps >> 1);
      if (ps & 1) dq_put(DSLOT, sBd, ps >> 1);
    }
  };

  // ---- pipeline. Per step this wave issues kStepLoads vector-memory operations: the B loads
  // of tile t+2, then the two A DMAs of tile t+3. Tiles past the end are re-reads of the last
  // tile into a stage nobody reads, so every step has the same count in flight. ----
  constexpr int kStepLoads = (GS ? 3 : 2) + 2;
  // vmcnt(2 * kStepLoads) expcnt(7) lgkmcnt(0): the A DMA of tile t (issued three steps ago)
  // landed, and this wave's LDS reads and B writes of the previous step are done.
  constexpr int kWaitTile = ((2 * kStepLoads) & 15) | (7 << 4) | (((2 * kStepLoads) >> 4) << 14);
  constexpr int kWaitPro = ((kStepLoads + 2) & 15) | (7 << 4) | (15 << 8);
  // prologue, in the order the waits count: B of tiles 0 and 1, A of tiles 0..2
  load_b(0, pk_int_c<0>{});
  __builtin_amdgcn_sched_barrier(0);
  issue_a_part(0, sA0, 0);
  issue_a_part(0, sA0, 1);
  issue_a_part(min(1, last), sA1, 0);
  issue_a_part(min(1, last), sA1, 1);
  __builtin_amdgcn_sched_barrier(0);
  load_b(min(1, last), pk_int_c<1>{});
  __builtin_amdgcn_sched_barrier(0);
  issue_a_part(min(2, last), sA2, 0);
  issue_a_part(min(2, last), sA2, 1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < 4; ++b) dq_put(pk_int_c<0>{}, sB0, b);
  __builtin_amdgcn_s_waitcnt(kWaitPro);  // tile 0's A DMA landed
  // Step kt: stage kt % 4 is multiplied; B loads of tile kt+2 go to slot kt % 2; tile kt+1's
  // B (slot (kt+1) % 2) is dequantised into stage (kt+1) % 4; tile kt+3's A DMA goes to stage
  // (kt+3) % 4, whose last reader was step kt-1 (before this step's barrier).
  auto step = [&](int kt, char* sAc, char* sBc, char* sBd, char* sAn, auto LS, auto DS) {
    __builtin_amdgcn_s_waitcnt(kWaitTile);
    asm volatile("s_barrier" ::: "memory");
    load_b(min(kt + 2, last), LS);
    __builtin_amdgcn_sched_barrier(0);
    compute(sAc, sBc, min(kt + 3, last), sAn, DS, sBd);
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + 3 < ktiles; kt += 4) {
    step(kt, sA0, sB0, sB1, sA3, pk_int_c<0>{}, pk_int_c<1>{});
    step(kt + 1, sA1, sB1, sB2, sA0, pk_int_c<1>{}, pk_int_c<0>{});
    step(kt + 2, sA2, sB2, sB3, sA1, pk_int_c<0>{}, pk_int_c<1>{});
    step(kt + 3, sA3, sB3, sB0, sA2, pk_int_c<1>{}, pk_int_c<0>{});
  }
  if (kt < ktiles) step(kt, sA0, sB0, sB1, sA3, pk_int_c<0>{}, pk_int_c<1>{});
  if (kt + 1 < ktiles) step(kt + 1, sA1, sB1, sB2, sA0, pk_int_c<1>{}, pk_int_c<0>{});
  if (kt + 2 < ktiles) step(kt + 2, sA2, sB2, sB3, sA1, pk_int_c<0>{}, pk_int_c<1>{});
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA into LDS outlives the waves
  mfma_drain();

  // ---- epilogue: C, scaled, in the output dtype ----
  char* const out_base = reinterpret_cast<char*>(p.c);
  const int64_t ld_out = p.ldc;
  const int out_dtype = p.c_dtype;
  const float oscale = p.scale;
  const int esz = out_dtype == PK_F32 ? 4 : 2;
  const int em = lane & 15, en = 4 * (lane >> 4);
  if ((ld_out * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(out_base) & 15) == 0) {
    // each wave stages 64-row halves of its 128 x 64 block in one 16 KB stage array (rows of
    // 64 values, 16-byte chunks XOR-swizzled by row), then writes them back row-contiguous
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS reads are done
    __syncthreads();                     // and every other wave's: the stages are free
    char* sW = wave == 0 ? sA0 : wave == 1 ? sA1 : wave == 2 ? sA2 : wave == 3 ? sA3
             : wave == 4 ? sB0 : wave == 5 ? sB1 : wave == 6 ? sB2 : sB3;
    with_dtype(out_dtype, [&](auto DT) {
      constexpr int dt = decltype(DT)::value;
      constexpr int E = dt == PK_F32 ? 4 : 2;
      constexpr int RB = WTN * E, NCH = RB / 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < GM / 2; ++ii)
#pragma unroll
          for (int j = 0; j < GN; ++j) {
            const int r = 16 * ii + em, col = 16 * j + en;
            const int byte = col * E;
            char* dst = sW + r * RB + ((((byte >> 4) ^ (r % NCH)) << 4) | (byte & 15));
            const pk_f4 v = acc[(GM / 2) * h + ii][j] * oscale;
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
        for (int c0 = 0; c0 < 64 * NCH; c0 += 64) {
          const int idx = c0 + lane, r = idx / NCH, ch = idx % NCH;
          const pk_u4v val = *reinterpret_cast<const pk_u4v*>(sW + r * RB + ((ch ^ (r % NCH)) << 4));
          const int gm = m0 + wm0 + 64 * h + r, gn = n0 + wn0 + ch * (16 / E);
          if (gm < p.M && gn < p.N)  // N % 8 == 0 and 16-byte chunks of 8 or 4 values
            *PK_GLOBAL(pk_u4v, out_base + ((int64_t)gm * ld_out + gn) * E) = val;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next half is staged
      }
    });
    return;
  }
  const bool vec = ld_out % 4 == 0 && (reinterpret_cast<uintptr_t>(out_base) & (4 * esz - 1)) == 0;
  with_dtype(out_dtype, [&](auto DT) {
    constexpr int dt = decltype(DT)::value;
#pragma unroll
    for (int i = 0; i < GM; ++i)
#pragma unroll
      for (int j = 0; j < GN; ++j) {
        const int gm = m0 + wm0 + 16 * i + em;
        const int gn = n0 + wn0 + 16 * j + en;  // N % 8 == 0: all four in or out
        if (gm < p.M && gn < p.N) store4_as<dt>(out_base, (int64_t)gm * ld_out + gn, acc[i][j] * oscale, vec);
      }
  });
}

bool w4_wide_ok(int M, int N, int K, int group, bool has_gs, int64_t lda, int64_t ldb) {
  if (M < 256 || N < 256 || N % 8 || K % 32 || K < 32) return false;
  if (has_gs && group % 32) return false;
  // 32-bit buffer offsets
  if ((int64_t)M * lda * 2 >= (1ll << 31)) return false;
  if ((int64_t)K * ldb * 4 >= (1ll << 31)) return false;
  return true;
}

int w4_wide_launch(const void* a, int64_t lda, const void* b, int64_t ldb, const void* scales,
                   int group, float scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                   hipStream_t s) {
  W4WideParams p;
  p.a = reinterpret_cast<const pk_half*>(a);
  p.lda = lda;
  p.b = reinterpret_cast<const uint32_t*>(b);
  p.ldb = ldb;
  p.scales = reinterpret_cast<const pk_half*>(scales);
  p.group = group > 0 ? group : K;
  p.scale = scale;
  p.c = c;
  p.c_dtype = c_dtype;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (int)cdiv(M, 256);
  p.tiles_n = (int)cdiv(N, 256);
  const dim3 grid(p.tiles_m * p.tiles_n);
  if (scales) gemm_w4_wide_kernel<true><<<grid, 512, 0, s>>>(p);
  else gemm_w4_wide_kernel<false><<<grid, 512, 0, s>>>(p);
  PK_LAUNCH_CHECK("w4a16 gemm (256 x 256)");
  return PK_OK;
}

}  // namespace pk
