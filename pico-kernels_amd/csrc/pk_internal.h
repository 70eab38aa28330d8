// Internal planning/launch interfaces shared between the kernel files and the C-ABI layer.
#pragma once
#include "pk_common.h"

namespace pk {

// C = scale * sum over slices of the (S, M, N) fp32 partials, in slice order.
int splitk_reduce(const float* partials, int S, int M, int N, float scale, void* c, int c_dtype,
                  int64_t ldc, hipStream_t s);

struct GemvPlan {
  int rpt, rl, split, k_slice, tiles;
  int mfma;  // 1: MFMA kernel eligible (k_slice and group multiples of 64)
};
bool gemv_plan(int M, int N, int K, int group, bool has_gs, int split_req, GemvPlan* out);
size_t gemv_workspace_bytes(const GemvPlan& pl, int M, int N);
// Launches the GEMV; with split > 1 the slices' partials go to `workspace` and, unless
// partials_only, the ordered reduction into C follows.
int gemv_launch(const GemvPlan& pl, const void* a, int64_t lda, const uint32_t* qw, int64_t ldq,
                const void* scales, int group, float tensor_scale, void* c, int c_dtype,
                int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only = false);

// W4A16 for kSkinnyMinM <= M <= kSkinnyMaxM (w4a16_skinny.hip): weights to registers, MFMA
// per 16 activation rows, 4-wave LDS reduction, split-K partials.
constexpr int kSkinnyMinM = 5;
constexpr int kSkinnyMaxM = 32;
struct SkinnyPlan {
  int mb;  // 16-row activation blocks (1 or 2)
  int split, k_slice, tiles;
};
bool skinny_plan(int M, int N, int K, int group, bool has_gs, int split_req, SkinnyPlan* out);
bool skinny_fits(int M, int N, int K, int64_t lda, int64_t ldq, int group, bool has_gs);
int skinny_launch(const SkinnyPlan& pl, const void* a, int64_t lda, const uint32_t* qw,
                  int64_t ldq, const void* scales, int group, float tensor_scale, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                  bool partials_only = false);

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
                int64_t ldb, const void* scales, int group, float tensor_scale, void* c,
                int c_dtype, int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only = false);

// Large-tile MFMA GEMMs (gemm_v2.hip).
bool v2_f16_ok(int M, int N, int K, int k_slice, int group, bool has_gs, int64_t lda, int64_t ldb,
               bool int4);
int v2_f16_launch(int bm, int bmode, const void* a, int64_t lda, const void* b, int64_t ldb,
                  const void* scales, int group, float scale, void* c, int c_dtype, int64_t ldc,
                  int M, int N, int K, int split, void* workspace, hipStream_t s,
                  bool partials_only);
int v2_f8_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s);

// 256 x 256 fp8 GEMM with a 4-stage DMA pipeline and transposing LDS reads for (K, N) B
// (gemm_f8_v3.hip).
bool f8_v3_ok(int M, int N, int K, int64_t lda, int64_t ldb, int b_layout, const void* b);
int f8_v3_launch(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                 float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                 hipStream_t s);

}  // namespace pk
