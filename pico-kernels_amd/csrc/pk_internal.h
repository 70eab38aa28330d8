// Internal planning/launch interfaces shared between the kernel files and the C-ABI layer.
#pragma once
#include <atomic>

#include "pk_common.h"

namespace pk {

// Workspace layout of pk_w4a16_gemm and pk_gemm_f16: the first kWsCounterBytes hold split-K
// arrival counters (one 128-byte line per column tile; zero before first use, left zero by
// every call); the fp32 partials of split-K slices follow.
constexpr size_t kWsCounterBytes = 64 << 10;
constexpr int kWsMaxTiles = (int)(kWsCounterBytes / 128);
inline float* ws_partials(void* ws) {
  return ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kWsCounterBytes) : nullptr;
}
inline unsigned* ws_counters(void* ws) { return reinterpret_cast<unsigned*>(ws); }
// Where a launcher writes split-K partials: after the counters of a workspace, or at the start
// of the caller's own partials buffer (the partials-only entry point).
inline float* split_partials(void* ws, bool partials_only) {
  return partials_only ? reinterpret_cast<float*>(ws) : ws_partials(ws);
}
// Where the packed int4 weight words live. Rows (gemm_int4.pack_int4_n's layout viewed as a
// (K, ldq) int32 array): word w of row k at k * ldq + w. Blocks (pk_w4a16_gemm_tiled): 128 rows
// x 256 columns (32 words) per 16 KB block, row-major inside, the blocks ordered by row block
// and then column tile -- word w of row k at ((k / 128) * T + w / 32) * 4096 + (k % 128) * 32 +
// w % 32, T = N / 256. A kernel reads a 16-byte chunk (four words of one column tile) at byte
//   (w / 32) * tile_bytes + (k / 128) * kblock_bytes + (k % 128) * row_bytes + (w % 32) * 4,
// which is k * ldq * 4 + w * 4 for rows. Every kernel's rows per address base stay inside one
// aligned 128-row block (the GEMV's 64-row wave groups, the register-dequant kernel's 32-row
// k-steps, the packed-B GEMM's 128-row k-tiles).
struct QLayout {
  int row_bytes;     // between consecutive rows inside a block: ldq * 4, or 128
  int tile_bytes;    // between consecutive 256-column tiles: 128, or 16 KB
  int kblock_bytes;  // between consecutive 128-row blocks: 128 * ldq * 4, or T * 16 KB
};
inline QLayout qlayout(bool tiled, int64_t ldq, int N) {
  return tiled ? QLayout{128, 16384, (N / 256) * 16384}
               : QLayout{(int)(ldq * 4), 128, (int)(128 * ldq * 4)};
}
// Byte offset of row k's words within its column tile.
__host__ __device__ __forceinline__ int qrow_off(const QLayout& q, int k) {
  return (k >> 7) * q.kblock_bytes + (k & 127) * q.row_bytes;
}

// Host: split-K slices may hand off through one XCD's L2 on the current device: its XCC
// count divides 8, PK_SPLITK_IN_L2 is not 0, and a probe launch (run once per device, at the
// first call from a stream that is not capturing; see splitk_reduce.hip) found every
// workgroup of a launch on XCD (b + c) mod that count. For a launch on `stream`.
bool splitk_in_l2_ok(hipStream_t stream);
// The same answer for queries that launch nothing (launch counts): the probe's result once it
// has run, before that the XCC-count and environment rule alone.
bool splitk_in_l2_possible();

// Host: allow `kernel` up to `bytes` of dynamic LDS on the current device. The attribute is
// set once per (device, kernel): `done` is a per-kernel bit set of the devices already done
// (64 at most); concurrent first calls may both set it, which is harmless.
int set_lds_limit_once(const void* kernel, int bytes, std::atomic<uint64_t>* done);

// C = scale * sum over slices of the (S, M, N) fp32 partials, in slice order. `small_groups`:
// workgroups of 64 threads instead of 256 (for 2, 4 or 8 slices), what the register-dequant
// kernel's partials reduce fastest with -- measured on MI355X, the whole call in graphs: with
// weights streamed from HBM (rotating copies) o_proj 4096 x 4096 M = 128 16.15 -> 15.6 us;
// with one cached weight copy 15.8 -> 12.9 us, M = 72 14.1 -> 12.7, 2048 x 2048 M = 128
// 13.0 -> 10.3 -- while after the packed-B GEMM's planes 256 stay faster (streamed weights:
// qkv M = 128 18.0 against 18.2, down 27.6 against 28.4; cached copy: qkv 18.7 against 19.0,
// down 26.6 against 27.6; 128 and 512 within 1% of 256).
int splitk_reduce(const float* partials, int S, int M, int N, OutEpi epi, void* c, int c_dtype,
                  int64_t ldc, hipStream_t s, bool small_groups = false);

struct GemvPlan {
  int rpt, rl, split, k_slice, tiles;
  int mfma;  // MFMA kernel row blocks per wave (k_slice = 256 * mfma); 0: VALU kernel
};
bool gemv_plan(int M, int N, int K, int group, bool has_gs, int split_req, GemvPlan* out);
size_t gemv_workspace_bytes(const GemvPlan& pl, int M, int N);
// Launches the GEMV; with split > 1 the slices' partials go to `workspace` and, unless
// partials_only, the ordered reduction into C follows.
// `tiled`: the weights are in blocks (QLayout; the MFMA kernel only, see gemv_tiled_ok).
int gemv_launch(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw, int64_t ldq,
                const void* scales, int group, OutEpi epi, void* c, int c_dtype,
                int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only = false, bool tiled = false);
// The plan and operands run the MFMA kernel, the one that reads blocks.
bool gemv_tiled_ok(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                   int64_t ldq, const void* scales, int group, int M, int N, int K);

// W4A16 decode GEMV on strip-layout weights (w4a16_strips.hip): 1 <= M <= 8, one workgroup
// per 16-column strip over the whole of K, one launch.
bool strips_shape_ok(int M, int N, int K, int group, bool has_gs);
int strips_launch(const void* a, int64_t lda, const uint8_t* qs, const void* ss, int group,
                  OutEpi epi, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                  hipStream_t stream);
bool strips_config_set(int blocks_per_wave);

// W4A16 for kSkinnyMinM <= M <= kSkinnyMaxM (w4a16_skinny.hip): weights to registers, MFMA
// per 16 activation rows, LDS reduction over the workgroup's waves, split-K partials.
constexpr int kSkinnyMinM = 5;
constexpr int kSkinnyMaxM = 128;
struct SkinnyPlan {
  int mb;         // 16-row activation blocks per workgroup (1, 2 or 4)
  int cpl, nw;    // columns per lane (16 or 8), waves per workgroup (4 or 8)
  int row_parts;  // workgroups along M per (column tile, slice)
  int split, k_slice, tiles;
  bool mg;        // a wave's rows span several 128-row groups (folded at each boundary)
};
// `tiled`: the plan for block-layout weights (QLayout): one 16-row block (M <= 16) takes
// 128-column tiles there (measured on MI355X: down M=8 15.3 -> 13.7 us, gate_up 13.1 -> 12.7).
bool skinny_plan(int M, int N, int K, int group, bool has_gs, int split_req, SkinnyPlan* out,
                 bool tiled = false);
// Fix the layout the plan uses (cpl 8 or 16, nw 4 or 8), or restore the automatic one (0, 0).
bool skinny_layout_set(int cpl, int nw);
bool skinny_fits(int M, int N, int K, int64_t lda, int64_t ldq, int group, bool has_gs);
// Split-K of the skinny kernel adds its slices in L2 inside the launch (one launch).
// `l2`: splitk_in_l2_ok(stream) for a launch, splitk_in_l2_possible() for a query.
bool skinny_l2(const SkinnyPlan& pl, bool l2);
size_t skinny_workspace_bytes(const SkinnyPlan& pl, int M, int N);
int skinny_launch(const SkinnyPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                  int64_t ldq, const void* scales, int group, OutEpi epi, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                  bool partials_only = false, bool tiled = false);

struct GemmCfg {
  int bm, bn, wm, wn;
};
struct GemmPlan {
  GemmCfg cfg;
  int split, k_slice, tiles_m, tiles_n;
};
bool gemm_plan(int M, int N, int K, int group, bool has_gs, int split_req, GemmPlan* out);
size_t gemm_workspace_bytes(const GemmPlan& pl, int M, int N);
int gemm_launch(const GemmPlan& pl, int bmode, const void* a, int64_t lda, const void* b,
                int64_t ldb, const void* scales, int group, OutEpi epi, void* c,
                int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only = false);

// Large-tile MFMA GEMMs (gemm_v2.hip).
bool v2_f16_ok(int M, int N, int K, int k_slice, int group, bool has_gs, int64_t lda, int64_t ldb,
               bool int4);
int v2_f16_launch(int bm, int bmode, const void* a, int64_t lda, const void* b, int64_t ldb,
                  const void* scales, int group, OutEpi epi, void* c, int c_dtype, int64_t ldc,
                  int M, int N, int K, int split, void* workspace, hipStream_t s,
                  bool partials_only);
int v2_f8_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s);

// W4A16 GEMM with the int4 B tile kept packed in LDS and read with transposing 4-bit reads,
// 128 x 256 tiles, eight waves splitting each k-tile in halves (w4a16_tr4.hip); N % 256 == 0,
// K % (128 * split) == 0; split > 1 writes fp32 partial planes and reduces them.
bool tr4_shape_ok(int M, int N, int K, int group, bool has_gs);
bool tr4_split_ok(int K, int split);
int tr4_pick_split(int M, int N, int K);
bool tr4_ok(int M, int N, int K, int group, bool has_gs, int64_t lda, const void* b, int64_t ldb,
            int64_t ldc, int c_dtype, const void* c, int split);
int tr4_launch(const void* a, int64_t lda, const void* b, int64_t ldb, const void* scales,
               int group, OutEpi epi, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
               int split, void* workspace, hipStream_t s, bool partials_only, bool tiled = false);

// 256 x 256 fp8 GEMM with a 4-stage DMA pipeline and transposing LDS reads for (K, N) B
// (gemm_f8_v3.hip).
bool f8_v3_ok(int M, int N, int K, int64_t lda, int64_t ldb, int b_layout, const void* b);
int f8_v3_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s);

}  // namespace pk
