// C ABI for the W4A16 matmul (gemm_int4.int4_gemm + the group-128 / split-K path) and the
// dense fp16 split-K matmul (gemm_splitk.triton_gemm_splitk).
//
// Dispatch: M <= 4 runs the HBM-bound GEMV (w4a16_gemv.hip); up to 64 rows the register-dequant
// MFMA kernel (w4a16_skinny.hip), except from 33 rows on layers of more than 4096 x 8192
// weights; larger M the GEMM that keeps B packed in LDS (w4a16_tr4.hip, split-K where its
// tiles leave CUs idle) where its shape rules hold, else the register-dequant kernel (up to
// 128 rows of layers of at most 4096 x 4096 weights) or the GEMMs that dequantise into LDS. All
// honour an explicit split_k. make_plan gives the measured rules.
#include "pk_internal.h"

#include <atomic>

using namespace pk;

namespace {

enum { kKernelGemv = 1, kKernelGemm = 2, kKernelSkinny = 3, kKernelGemmTr4 = 4 };

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_w4a16(const void* a, int64_t lda, const uint32_t* qw, int64_t ldq, const void* scales,
                int group_size, const void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                int split_k) {
  PK_REQUIRE(a != nullptr && qw != nullptr && c != nullptr, "pk_w4a16_gemm: null pointer");
  PK_REQUIRE(M >= 1 && N >= 1 && K >= 1, "pk_w4a16_gemm: empty shape M=%d N=%d K=%d", M, N, K);
  PK_REQUIRE(N % 8 == 0, "pk_w4a16_gemm: N=%d must be a multiple of 8 (one int32 word)", N);
  PK_REQUIRE(K % 32 == 0, "pk_w4a16_gemm: K=%d must be a multiple of 32", K);
  PK_REQUIRE(lda >= K && lda % 8 == 0 && aligned16(a),
             "pk_w4a16_gemm: A rows must be 16-byte aligned (lda=%lld)", (long long)lda);
  PK_REQUIRE(ldq >= N / 8, "pk_w4a16_gemm: ldq=%lld < N/8", (long long)ldq);
  PK_REQUIRE(ldc >= N, "pk_w4a16_gemm: ldc < N");
  PK_REQUIRE(c_dtype == PK_F32 || c_dtype == PK_F16 || c_dtype == PK_BF16,
             "pk_w4a16_gemm: output dtype %d", c_dtype);
  PK_REQUIRE(split_k >= 0, "pk_w4a16_gemm: split_k must be >= 0");
  if (scales != nullptr) {
    PK_REQUIRE(group_size >= 32 && group_size % 32 == 0 && K % group_size == 0,
               "pk_w4a16_gemm: group_size=%d must be a multiple of 32 dividing K=%d",
               group_size, K);
    PK_REQUIRE(aligned16(scales), "pk_w4a16_gemm: scales must be 16-byte aligned");
  }
  return PK_OK;
}

struct W4Plan {
  int kernel;
  int tr4_split;  // kKernelGemmTr4: its split (gemm holds the same split for the fallback)
  GemvPlan gemv;
  GemmPlan gemm;
  SkinnyPlan skinny;
};

bool make_plan(int M, int N, int K, int group_size, bool has_gs, int split_k, W4Plan* pl,
               bool tiled = false) {
  if (M <= 4 && gemv_plan(M, N, K, group_size, has_gs, split_k, &pl->gemv)) {
    pl->kernel = kKernelGemv;
    return true;
  }
  // 65..128 rows of a layer of 1024^2 .. 4096^2 weights: two row parts of the register-dequant
  // kernel where its automatic plan needs at most 8 slices (measured on MI355X at M = 72, 96
  // and 128 against the packed-B GEMM: 4096 x 4096 18.8 -> 15.6 us at M = 128, the 1024..4096
  // layers 5-21% faster; with 16 slices, K = 4096 x N = 1024, 21-27% slower).
  if (M > 64 && split_k == 0 && (int64_t)K * N >= 1024ll * 1024 &&
      skinny_plan(M, N, K, group_size, has_gs, 0, &pl->skinny, tiled) && pl->skinny.split <= 8 &&
      gemm_plan(M, N, K, group_size, has_gs, pl->skinny.split, &pl->gemm)) {
    pl->kernel = kKernelSkinny;
    return true;
  }
  // Above the skinny kernel's 64 rows, and from 33 rows on layers of more than 4096 x 8192
  // weights with an automatic split: the packed-B GEMM where its shape rules hold, with the
  // GEMM that dequantises into LDS at the same split as its fallback (operands misaligned for
  // it, or beyond its 32-bit offsets), so the workspace covers both. (33..64 rows, measured on
  // MI355X: 4096 x 11008, 4096 x 14336 and 14336 x 4096 3-16% faster on the packed-B GEMM;
  // 4096 x 6144, 4096 x 8192, 8192 x 4096 and 14336 x 2048 9-35% faster on the skinny kernel.)
  const bool tr4_rows = M > 64 || (M > 32 && split_k == 0 && (int64_t)K * N > 4096ll * 8192);
  if (tr4_rows && tr4_shape_ok(M, N, K, group_size, has_gs)) {
    const int s = split_k > 0 ? split_k : tr4_pick_split(M, N, K);
    if (tr4_split_ok(K, s) && gemm_plan(M, N, K, group_size, has_gs, s, &pl->gemm)) {
      pl->kernel = kKernelGemmTr4;
      pl->tr4_split = s;
      return true;
    }
  }
  // The skinny kernel's split must also be one the GEMM accepts: the GEMM is its fallback
  // when a buffer exceeds 32-bit offsets, and the workspace size is the same (split*M*N*4).
  if (skinny_plan(M, N, K, group_size, has_gs, split_k, &pl->skinny, tiled) &&
      gemm_plan(M, N, K, group_size, has_gs, pl->skinny.split, &pl->gemm)) {
    pl->kernel = kKernelSkinny;
    return true;
  }
  if (gemm_plan(M, N, K, group_size, has_gs, split_k, &pl->gemm)) {
    pl->kernel = kKernelGemm;
    return true;
  }
  return false;
}

int plan_split(const W4Plan& pl) {
  return pl.kernel == kKernelGemv ? pl.gemv.split
         : pl.kernel == kKernelSkinny ? pl.skinny.split
                                      : pl.gemm.split;
}

size_t plan_ws(const W4Plan& pl, int M, int N) {
  if (pl.kernel == kKernelGemv) return gemv_workspace_bytes(pl.gemv, M, N);
  const size_t g = gemm_workspace_bytes(pl.gemm, M, N);
  if (pl.kernel != kKernelSkinny) return g;
  // the skinny kernel's tile-padded partials, or its GEMM fallback's (same split)
  const size_t k = skinny_workspace_bytes(pl.skinny, M, N);
  return k > g ? k : g;
}

// The kernel the plan runs reads block-layout weights (the GEMV's MFMA form, the register-
// dequant kernel, the packed-B GEMM) and its launch conditions hold, so no fallback to a
// rows-only kernel can happen.
bool plan_reads_tiles(const W4Plan& pl, const void* a, int64_t lda, const uint32_t* qw,
                      int64_t ldq, const void* scales, int group, const void* c, int c_dtype,
                      int64_t ldc, int M, int N, int K) {
  if (pl.kernel == kKernelGemv) return gemv_tiled_ok(pl.gemv, a, lda, qw, ldq, scales, group, M, N, K);
  if (pl.kernel == kKernelSkinny) return skinny_fits(M, N, K, lda, ldq, group, scales != nullptr);
  if (pl.kernel == kKernelGemmTr4)
    return tr4_ok(M, N, K, group, scales != nullptr, lda, qw, ldq, ldc, c_dtype, c, pl.tr4_split);
  return false;
}

int plan_launch(const W4Plan& pl, const void* a, int64_t lda, const uint32_t* qw, int64_t ldq,
                const void* scales, int group, OutEpi epi, void* c, int c_dtype,
                int64_t ldc, int M, int N, int K, void* workspace, hipStream_t s,
                bool partials_only, bool tiled = false) {
  if (pl.kernel == kKernelGemv)
    return gemv_launch(pl.gemv, a, lda, qw, ldq, scales, group, epi, c, c_dtype, ldc,
                       M, N, K, workspace, s, partials_only, tiled);
  if (pl.kernel == kKernelSkinny && skinny_fits(M, N, K, lda, ldq, group, scales != nullptr))
    return skinny_launch(pl.skinny, a, lda, qw, ldq, scales, group, epi, c, c_dtype,
                         ldc, M, N, K, workspace, s, partials_only, tiled);
  if (pl.kernel == kKernelGemmTr4 &&
      tr4_ok(M, N, K, group, scales != nullptr, lda, qw, ldq, ldc, c_dtype, c, pl.tr4_split))
    return tr4_launch(a, lda, qw, ldq, scales, group, epi, c, c_dtype, ldc, M, N, K,
                      pl.tr4_split, workspace, s, partials_only, tiled);
  if (tiled) {
    set_error("pk_w4a16_gemm_tiled: no kernel reads block-layout weights for M=%d N=%d K=%d", M, N, K);
    return PK_EUNSUPPORTED;
  }
  return gemm_launch(pl.gemm, 1, a, lda, qw, ldq, scales, group, epi, c, c_dtype, ldc,
                     M, N, K, workspace, s, partials_only);
}

}  // namespace

extern "C" int pk_w4a16_plan(int M, int N, int K, int group_size, int split_k, int* kernel_id,
                             int* split_used) {
  W4Plan pl;
  const bool has_gs = group_size > 0;
  if (!make_plan(M, N, K, has_gs ? group_size : K, has_gs, split_k, &pl)) {
    set_error("pk_w4a16_plan: no kernel for M=%d N=%d K=%d group=%d split_k=%d", M, N, K,
              group_size, split_k);
    return PK_EUNSUPPORTED;
  }
  // (kKernelGemmTr4 assumes operands aligned for it: misaligned ones run kKernelGemm)
  if (kernel_id) *kernel_id = pl.kernel;
  if (split_used) *split_used = plan_split(pl);
  return PK_OK;
}

extern "C" int pk_w4a16_skinny_layout(int cols_per_lane, int waves) {
  PK_REQUIRE(skinny_layout_set(cols_per_lane, waves),
             "pk_w4a16_skinny_layout: (%d, %d) is not (0, 0), or 8 or 16 columns per lane with 4 "
             "or 8 waves", cols_per_lane, waves);
  return PK_OK;
}

extern "C" int pk_w4a16_launches(int M, int N, int K, int group_size, int split_k) {
  W4Plan pl;
  const bool has_gs = group_size > 0;
  if (!make_plan(M, N, K, has_gs ? group_size : K, has_gs, split_k, &pl)) {
    set_error("pk_w4a16_launches: no kernel for M=%d N=%d K=%d group=%d split_k=%d", M, N, K,
              group_size, split_k);
    return PK_EUNSUPPORTED;
  }
  const int split = plan_split(pl);
  if (split <= 1) return 1;
  const bool l2 = pl.kernel == kKernelGemv
                      ? splitk_in_l2_possible() && pl.gemv.mfma && pl.gemv.tiles <= kWsMaxTiles
                      : pl.kernel == kKernelSkinny && skinny_l2(pl.skinny, splitk_in_l2_possible());
  return l2 ? 1 : 2;
}

extern "C" size_t pk_w4a16_workspace_bytes(int M, int N, int K, int group_size, int split_k) {
  W4Plan pl;
  const bool has_gs = group_size > 0;
  const int group = has_gs ? group_size : K;
  if (!make_plan(M, N, K, group, has_gs, split_k, &pl)) return 0;
  size_t need = plan_ws(pl, M, N);
  // enough for pk_w4a16_gemm_tiled's plan as well, where blocks are possible
  W4Plan pt;
  if (N % 256 == 0 && K % 256 == 0 && make_plan(M, N, K, group, has_gs, split_k, &pt, true)) {
    const size_t t = plan_ws(pt, M, N);
    if (t > need) need = t;
  }
  return need;
}

namespace {
// Activations whose rows span 2 GiB or more exceed the 32-bit buffer offsets of the kernels
// that read block-layout weights at large M (the packed-B GEMM). Such calls run as equal
// chunks of rows, each a whole multiple of 128 rows below that limit (0: lda too large).
constexpr int64_t kBufferBytes = 1ll << 31;
int64_t tiled_rows_per_call(int64_t M, int64_t lda) {
  if (M * lda * 2 < kBufferBytes) return M;
  const int64_t cap = ((kBufferBytes - 1) / (lda * 2)) / 128 * 128;
  if (cap < 128) return 0;
  const int64_t chunks = cdiv(M, cap);
  return cdiv(cdiv(M, chunks), 128) * 128;
}

int w4a16_gemm_ws(const char* name, const void* a, int64_t lda, const uint32_t* qweight,
                  int64_t ldq, const void* scales, int group_size, OutEpi epi, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, int split_k, void* workspace,
                  size_t workspace_bytes, void* stream, bool tiled = false) {
  int rc = check_w4a16(a, lda, qweight, ldq, scales, group_size, c, c_dtype, ldc, M, N, K,
                       split_k);
  if (rc != PK_OK) return rc;
  if (tiled && (int64_t)M * lda * 2 >= kBufferBytes) {
    const int64_t rows = tiled_rows_per_call(M, lda);
    PK_REQUIRE(rows > 0, "%s: activation rows of %lld elements are beyond the block-layout "
               "kernels' 2 GiB buffers", name, (long long)lda);
    const int esz = c_dtype == PK_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < M; r0 += rows) {
      const int m = (int)(M - r0 < rows ? M - r0 : rows);
      rc = w4a16_gemm_ws(name, static_cast<const char*>(a) + r0 * lda * 2, lda, qweight, ldq,
                         scales, group_size, epi, static_cast<char*>(c) + r0 * ldc * esz,
                         c_dtype, ldc, m, N, K, split_k, workspace, workspace_bytes, stream,
                         true);
      if (rc != PK_OK) return rc;
    }
    return PK_OK;
  }
  const bool has_gs = scales != nullptr;
  const int group = has_gs ? group_size : K;
  W4Plan pl;
  if (!make_plan(M, N, K, group, has_gs, split_k, &pl, tiled)) {
    set_error("%s: split_k=%d does not divide K=%d into slices of whole groups "
              "(group %d, multiple of 32 rows)", name, split_k, K, group);
    return PK_EINVAL;
  }
  if (tiled && !plan_reads_tiles(pl, a, lda, qweight, ldq, scales, group, c, c_dtype, ldc, M, N, K)) {
    set_error("%s: no kernel reads block-layout weights for M=%d N=%d K=%d split_k=%d (the plan "
              "picked kernel %d, or its operands are misaligned)", name, M, N, K, split_k, pl.kernel);
    return PK_EUNSUPPORTED;
  }
  const size_t need = plan_ws(pl, M, N);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("%s: workspace of %zu bytes needed (got %zu)", name, need, workspace_bytes);
    return PK_EWORKSPACE;
  }
  return plan_launch(pl, a, lda, qweight, ldq, scales, group, epi, c, c_dtype, ldc, M, N, K,
                     workspace, (hipStream_t)stream, false, tiled);
}
}  // namespace

extern "C" int pk_w4a16_gemm(const void* a, int64_t lda, const uint32_t* qweight, int64_t ldq,
                             const void* scales, int group_size, float tensor_scale, void* c,
                             int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return w4a16_gemm_ws("pk_w4a16_gemm", a, lda, qweight, ldq, scales, group_size,
                       OutEpi(tensor_scale), c, c_dtype, ldc, M, N, K, split_k, workspace,
                       workspace_bytes, stream);
}

extern "C" int64_t pk_w4a16_tiled_rows_per_call(int64_t M, int64_t lda) {
  return M >= 1 && lda >= 1 ? tiled_rows_per_call(M, lda) : 0;
}

extern "C" int pk_w4a16_gemm_tiled(const void* a, int64_t lda, const uint32_t* qtiled,
                                   const void* scales, int group_size, float tensor_scale,
                                   const void* bias, int bias_dtype, void* c, int c_dtype,
                                   int64_t ldc, int M, int N, int K, int split_k,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  PK_REQUIRE(N % 256 == 0 && K % 256 == 0,
             "pk_w4a16_gemm_tiled: blocks need N %% 256 == 0 and K %% 256 == 0 (N=%d K=%d)",
             N, K);
  PK_REQUIRE(scales == nullptr || group_size % 64 == 0,
             "pk_w4a16_gemm_tiled: group_size=%d must be a multiple of 64", group_size);
  PK_REQUIRE(qtiled != nullptr && aligned16(qtiled), "pk_w4a16_gemm_tiled: weights must be 16-byte aligned");
  PK_REQUIRE(bias == nullptr || bias_dtype == PK_F32 || bias_dtype == PK_F16 ||
                 bias_dtype == PK_BF16,
             "pk_w4a16_gemm_tiled: bias dtype %d", bias_dtype);
  return w4a16_gemm_ws("pk_w4a16_gemm_tiled", a, lda, qtiled, N / 8, scales, group_size,
                       OutEpi(tensor_scale, bias, bias_dtype), c, c_dtype, ldc, M, N, K,
                       split_k, workspace, workspace_bytes, stream, true);
}

extern "C" int pk_w4a16_gemm_bias(const void* a, int64_t lda, const uint32_t* qweight,
                                  int64_t ldq, const void* scales, int group_size,
                                  float tensor_scale, const void* bias, int bias_dtype, void* c,
                                  int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  PK_REQUIRE(bias == nullptr || bias_dtype == PK_F32 || bias_dtype == PK_F16 ||
                 bias_dtype == PK_BF16,
             "pk_w4a16_gemm_bias: bias dtype %d", bias_dtype);
  return w4a16_gemm_ws("pk_w4a16_gemm_bias", a, lda, qweight, ldq, scales, group_size,
                       OutEpi(tensor_scale, bias, bias_dtype), c, c_dtype, ldc, M, N, K,
                       split_k, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------------------
// pk_w4a16_gemm without a caller workspace, for callers that cannot allocate: the split-K
// workspace (arrival counters, then fp32 partials) is this file-scope device array. Each GPU
// holds its own copy, zero at load; every call leaves the counters zero again. Calls that
// overlap in time on one GPU share it and race.
// ---------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = 16u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Clears the split-K arrival counters at the head of the scratch array (a kernel, not a
// memset node, so the call can sit in a captured graph).
__global__ void noalloc_zero_counters(unsigned* counters, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) counters[i] = 0u;
}

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per device (the
// symbol's host-side name is not a device address); the first lookup also clears the
// counters on `stream`, ahead of the call that needs them.
int scratch_on_current_device(void** out, hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pk::hip_status(e, "pk_w4a16_gemm_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("pk_w4a16_gemm_noalloc: device %d beyond the %d this library tracks", dev, kMaxDevices);
    return PK_EUNSUPPORTED;
  }
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return pk::hip_status(e, "pk_w4a16_gemm_noalloc: hipGetSymbolAddress");
    if (ptr == nullptr) {
      set_error("pk_w4a16_gemm_noalloc: no device address for the scratch array");
      return PK_EHIP;
    }
    noalloc_zero_counters<<<16, 256, 0, stream>>>(static_cast<unsigned*>(ptr),
                                                   (int)(kWsCounterBytes / sizeof(unsigned)));
    e = hipGetLastError();
    if (e != hipSuccess) return pk::hip_status(e, "pk_w4a16_gemm_noalloc: counter clear");
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return PK_OK;
}
}  // namespace

extern "C" size_t pk_w4a16_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int pk_w4a16_gemm_noalloc(const void* a, int64_t lda, const uint32_t* qweight,
                                     int64_t ldq, const void* scales, int group_size,
                                     float tensor_scale, void* c, int c_dtype, int64_t ldc, int M,
                                     int N, int K, int split_k, void* stream) {
  int rc = check_w4a16(a, lda, qweight, ldq, scales, group_size, c, c_dtype, ldc, M, N, K,
                       split_k);
  if (rc != PK_OK) return rc;
  const bool has_gs = scales != nullptr;
  const int group = has_gs ? group_size : K;
  W4Plan pl;
  if (!make_plan(M, N, K, group, has_gs, split_k, &pl)) {
    set_error("pk_w4a16_gemm_noalloc: split_k=%d does not divide K=%d into slices of whole "
              "groups (group %d, multiple of 32 rows)", split_k, K, group);
    return PK_EINVAL;
  }
  size_t need = plan_ws(pl, M, N);
  // An automatic packed-B split whose partials exceed the array: the largest smaller split
  // that fits (an explicit split_k is taken as given).
  if (split_k == 0 && pl.kernel == kKernelGemmTr4 && need > kNoAllocScratchBytes) {
    for (int sp = pl.tr4_split - 1; sp >= 1; --sp) {
      W4Plan alt;
      if (!tr4_split_ok(K, sp) || !make_plan(M, N, K, group, has_gs, sp, &alt)) continue;
      const size_t alt_need = plan_ws(alt, M, N);
      if (alt_need <= kNoAllocScratchBytes) {
        pl = alt;
        need = alt_need;
        break;
      }
    }
  }
  if (need > kNoAllocScratchBytes) {
    set_error("pk_w4a16_gemm_noalloc: this shape and split need %zu bytes of split-K scratch, "
              "above the library's fixed %zu (use pk_w4a16_gemm with a workspace, or a smaller "
              "split)", need, kNoAllocScratchBytes);
    return PK_EWORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_on_current_device(&ws, (hipStream_t)stream);
    if (rc != PK_OK) return rc;
  }
  return plan_launch(pl, a, lda, qweight, ldq, scales, group, tensor_scale, c, c_dtype, ldc, M,
                     N, K, ws, (hipStream_t)stream, false);
}

extern "C" size_t pk_gemm_f16_workspace_bytes(int M, int N, int K, int split_k) {
  GemmPlan pl;
  if (!gemm_plan(M, N, K, K, false, split_k, &pl)) return 0;
  return gemm_workspace_bytes(pl, M, N);
}

// Dense C = A @ B for fp16 (bmode 0) or bf16 (bmode 2) operands.
static int gemm_dense(const char* name, int bmode, const void* a, int64_t lda, const void* b,
                      int64_t ldb, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                      int split_k, void* workspace, size_t workspace_bytes, void* stream) {
  PK_REQUIRE(a != nullptr && b != nullptr && c != nullptr, "%s: null pointer", name);
  PK_REQUIRE(M >= 1 && N >= 1 && K >= 1, "%s: empty shape", name);
  PK_REQUIRE(N % 8 == 0 && K % 32 == 0, "%s: needs N %% 8 == 0 and K %% 32 == 0", name);
  PK_REQUIRE(lda >= K && lda % 8 == 0 && aligned16(a), "%s: A rows must be 16-byte aligned", name);
  PK_REQUIRE(ldb >= N && ldb % 8 == 0 && aligned16(b), "%s: B rows must be 16-byte aligned", name);
  PK_REQUIRE(c_dtype == PK_F32 || c_dtype == PK_F16 || c_dtype == PK_BF16, "%s: out dtype", name);
  PK_REQUIRE(split_k >= 0, "%s: split_k must be >= 0", name);
  GemmPlan pl;
  if (!gemm_plan(M, N, K, K, false, split_k, &pl)) {
    set_error("%s: split_k=%d must divide K=%d into slices that are multiples of 64", name,
              split_k, K);
    return PK_EINVAL;
  }
  const size_t need = gemm_workspace_bytes(pl, M, N);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("%s: workspace of %zu bytes needed (got %zu)", name, need, workspace_bytes);
    return PK_EWORKSPACE;
  }
  return gemm_launch(pl, bmode, a, lda, b, ldb, nullptr, K, 1.0f, c, c_dtype, ldc, M, N, K,
                     workspace, (hipStream_t)stream);
}

extern "C" int pk_gemm_f16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                           int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                           void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_dense("pk_gemm_f16", 0, a, lda, b, ldb, c, c_dtype, ldc, M, N, K, split_k,
                    workspace, workspace_bytes, stream);
}

extern "C" int pk_gemm_bf16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                            int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_dense("pk_gemm_bf16", 2, a, lda, b, ldb, c, c_dtype, ldc, M, N, K, split_k,
                    workspace, workspace_bytes, stream);
}

extern "C" int pk_w4a16_gemm_partials(const void* a, int64_t lda, const uint32_t* qweight,
                                      int64_t ldq, const void* scales, int group_size,
                                      float* partials, size_t partials_bytes, int M, int N, int K,
                                      int split_k, void* stream) {
  int rc = check_w4a16(a, lda, qweight, ldq, scales, group_size, partials, PK_F32, N, M, N, K,
                       split_k);
  if (rc != PK_OK) return rc;
  const bool has_gs = scales != nullptr;
  const int group = has_gs ? group_size : K;
  W4Plan pl;
  if (!make_plan(M, N, K, group, has_gs, split_k, &pl)) {
    set_error("pk_w4a16_gemm_partials: no plan for split_k=%d, K=%d", split_k, K);
    return PK_EINVAL;
  }
  const int split = plan_split(pl);
  PK_REQUIRE(split >= 2, "pk_w4a16_gemm_partials: the plan has no split (split=%d)", split);
  const size_t need = (size_t)split * M * N * sizeof(float);
  if (partials_bytes < need) {
    set_error("pk_w4a16_gemm_partials: %zu bytes of partials needed (got %zu)", need, partials_bytes);
    return PK_EWORKSPACE;
  }
  return plan_launch(pl, a, lda, qweight, ldq, scales, group, 1.0f, nullptr, PK_F32, N, M, N,
                     K, partials, (hipStream_t)stream, true);
}

extern "C" int pk_splitk_reduce(const float* partials, int split, int M, int N, float scale,
                                void* c, int c_dtype, int64_t ldc, void* stream) {
  PK_REQUIRE(partials != nullptr && c != nullptr, "pk_splitk_reduce: null pointer");
  PK_REQUIRE(split >= 1 && M >= 1 && N >= 1 && N % 8 == 0, "pk_splitk_reduce: bad shape");
  PK_REQUIRE(ldc >= N, "pk_splitk_reduce: ldc < N");
  PK_REQUIRE(c_dtype == PK_F32 || c_dtype == PK_F16 || c_dtype == PK_BF16,
             "pk_splitk_reduce: output dtype %d", c_dtype);
  PK_REQUIRE((reinterpret_cast<uintptr_t>(partials) & 15) == 0, "pk_splitk_reduce: partials alignment");
  return splitk_reduce(partials, split, M, N, scale, c, c_dtype, ldc, (hipStream_t)stream);
}
