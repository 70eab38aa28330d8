/*
 * pico_kernels_amd.h -- C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * This is the drop-in boundary for the quantized-matmul path of pico-kernels. In the
 * reference, the operator API is a set of module-level Python functions that launch Triton
 * kernels; each entry point below names the reference function it replaces (file:line in
 * the reference repository). The Python modules gemm_int4.py / gemm_fp8.py / gemm_splitk.py
 * / quantize.py in pico-kernels_amd/ keep the reference signatures and call these symbols
 * through ctypes.
 *
 * Conventions
 *  - Plain pointers and sizes only. Device pointers are HIP device memory; `stream` is a
 *    hipStream_t passed as void* (NULL = the default stream). All launches are asynchronous
 *    on `stream`; nothing here synchronises the device.
 *  - The library never allocates device memory. Entry points that need scratch space take
 *    a caller-owned `workspace` whose size is given by the matching *_workspace_bytes().
 *    The workspace of pk_w4a16_gemm / pk_gemm_f16 starts with 64 KiB of split-K arrival
 *    counters: zero-fill a workspace once when it is allocated; every call leaves the
 *    counters zero again, so one workspace serves any sequence of shapes. (pk_absmax's
 *    workspace needs no initialisation.) Calls ordered on one stream may reuse a
 *    workspace; calls that overlap in time must not share one.
 *  - Matrices are row-major with an explicit leading dimension (elements, or 32-bit words
 *    for packed int4).
 *  - Return value: PK_OK (0) or a negative PK_E* code; pk_last_error() then describes the
 *    failure (thread-local, valid until the next failing call on the same thread).
 */
#ifndef PICO_KERNELS_AMD_H
#define PICO_KERNELS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum {
  PK_F32 = 0,
  PK_F16 = 1,
  PK_BF16 = 2,
  PK_E4M3 = 3, /* OCP fp8 e4m3 ("e4m3fn"), one byte */
  PK_I8 = 4,
  PK_U8 = 5,
  PK_I32 = 6
};

/* Status codes. */
enum {
  PK_OK = 0,
  PK_EINVAL = -1,       /* bad argument: shape, dtype, alignment, null pointer */
  PK_EUNSUPPORTED = -2, /* valid request this build does not implement */
  PK_EWORKSPACE = -3,   /* workspace missing or too small */
  PK_EHIP = -4          /* a HIP runtime call failed (launch error) */
};

/* Library version (major*10000 + minor*100 + patch). */
int pk_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* pk_last_error(void);

/* ------------------------------------------------------------------------------------- */
/* Reductions and casts                                                                  */
/* ------------------------------------------------------------------------------------- */

/* out_dev[0] = max(|x|) over n elements as fp32 (NaN if any element is NaN).
 * Replaces `w.abs().max()` in gemm_int4.quantize_int4 (gemm_int4.py:60) and
 * `x.abs().max()` in gemm_fp8.quantize (gemm_fp8.py:94). */
size_t pk_absmax_workspace_bytes(int64_t n);
int pk_absmax(const void* x, int x_dtype, int64_t n, float* out_dev, void* workspace,
              size_t workspace_bytes, void* stream);

/* Per-tensor int4 codes: q[i] = int8(clamp(round(T(x[i] / scale)), -8, 7)) where T rounds
 * the fp32 quotient to x's dtype (fp16/bf16) exactly as a torch tensor op does, round is
 * half-to-even, and `scale` is the Python float narrowed to fp32. A NaN quotient gives 0.
 * Replaces gemm_int4.quantize_int4 (gemm_int4.py:58-62); the scale itself
 * (absmax / 7.0 in double) is computed by the caller from pk_absmax. */
int pk_quantize_int4(const void* w, int w_dtype, int64_t n, float scale, int8_t* q,
                     void* stream);

/* Pack int4 codes two per byte along N: packed[k, j] = (q[k,2j] & 0xF) | (q[k,2j+1] << 4).
 * q is (rows, cols) int8 with row stride ldq elements; packed is (rows, cols/2) contiguous.
 * cols must be even. Replaces gemm_int4.pack_int4_n (gemm_int4.py:65-72). */
int pk_pack_int4(const int8_t* q, int64_t rows, int64_t cols, int64_t ldq, uint8_t* packed,
                 void* stream);

/* Inverse of pk_pack_int4 with sign extension (codes in [-8, 7]). Mirrors the in-kernel
 * unpack of gemm_int4.int4_gemm_kernel (gemm_int4.py:44-49). */
int pk_unpack_int4(const uint8_t* packed, int64_t rows, int64_t cols, int8_t* q,
                   void* stream);

/* Group-wise symmetric round-to-nearest quantization along K of a (K, N) weight, the
 * arithmetic of quantize.rtn_layer / quantize_col (quantize.py:42-68): for every column n
 * and every group of `group_size` consecutive rows (the last group may be short),
 *   s = max(max|w|, 1e-12) / qmax  (fp32),  q = clamp(round(w / s), -qmax, qmax),
 * with qmax = 2^(bits-1) - 1 and all arithmetic in fp32 (w widened exactly).
 * group_size <= 0 means one group per column (quantize_col with group_size=None).
 * Outputs (each may be NULL):
 *   qweight   (K, N/8) int32: 4-bit codes, byte-identical to pack_int4_n (bits must be 4,
 *             N % 8 == 0)
 *   scales    (ceil(K/G), N) in `scale_dtype` (PK_F16 or PK_F32), RNE-rounded from s
 *   fake      (K, N) in `fake_dtype`: T(q * s), the tensor rtn_layer returns
 * half_math != 0 reproduces quantize_col applied directly to an fp16 tensor (every op
 * rounded to fp16, the 1e-12 floor becoming 0); it requires w_dtype == PK_F16.
 * Replaces quantize.rtn_layer / quantize.quantize_col (quantize.py:42-68) and is the
 * producer of the packed group-128 format consumed by pk_w4a16_gemm. */
int pk_quantize_group(const void* w, int w_dtype, int64_t K, int64_t N, int64_t ldw, int bits,
                      int group_size, int half_math, uint32_t* qweight, void* scales,
                      int scale_dtype, void* fake, int fake_dtype, void* stream);

/* Scaled cast to fp8 e4m3: out[i] = e4m3(T(x[i] * scale)) where T rounds the fp32 product to
 * x's dtype (fp16/bf16/fp32), then round-to-nearest-even, non-saturating (overflow -> NaN).
 * Replaces `(x * scale).to(torch.float8_e4m3fn)` in gemm_fp8.quantize (gemm_fp8.py:95). */
int pk_cast_e4m3(const void* x, int x_dtype, int64_t n, float scale, uint8_t* out,
                 void* stream);

/* ------------------------------------------------------------------------------------- */
/* W4A16 matmul                                                                          */
/* ------------------------------------------------------------------------------------- */

/* C[M,N] = tensor_scale * sum_k A[m,k] * Wdq[k,n] with fp32 accumulation, where
 *   Wdq[k,n] = q[k,n] * S[k / group_size, n]   (scales given; fp16, row stride N)
 *   Wdq[k,n] = q[k,n]                          (scales == NULL: per-tensor mode)
 * A is fp16 (M, K) with row stride lda; qweight is (K, N/8) int32 with row stride ldq words,
 * nibble i of word j holding column 8j+i (pack_int4_n byte order); C is fp32/fp16/bf16 with
 * row stride ldc. Requires N % 8 == 0, K % 32 == 0 and, with scales, K % group_size == 0
 * and group_size % 32 == 0.
 * split_k: 0 = choose automatically; s >= 1 = split K into s contiguous slices of K/s rows
 * (K/s a multiple of 8 for M <= 4, of 64 otherwise) whose fp32 partial sums are reduced in a
 * fixed order (results are bitwise reproducible run to run).
 * workspace: pk_w4a16_workspace_bytes() bytes, zero-filled once at allocation (split-K
 * arrival counters, then fp32 partials of the slices). For M <= 16 on MI355X (M <= 32 on
 * layers of at most 4096 x 6144 weights) the slices of a column tile are placed on one XCD
 * and the last to finish adds them through that XCD's L2, in the same fixed order as
 * pk_splitk_reduce (bitwise the same result), so no second launch is needed; larger M adds
 * them with a pk_splitk_reduce launch (pk_w4a16_launches reports which).
 * Replaces gemm_int4.int4_gemm (gemm_int4.py:75-92, per-tensor mode, the `c * scale`
 * epilogue fused) and provides the group-128 / split-K W4A16 path; the split-K semantics
 * (contiguous K slices of K / split_k) follow gemm_splitk.triton_gemm_splitk
 * (gemm_splitk.py:49-53, 67-80) without its fp32 atomics. */
size_t pk_w4a16_workspace_bytes(int M, int N, int K, int group_size, int split_k);
int pk_w4a16_gemm(const void* a, int64_t lda, const uint32_t* qweight, int64_t ldq,
                  const void* scales, int group_size, float tensor_scale, void* c,
                  int c_dtype, int64_t ldc, int M, int N, int K, int split_k, void* workspace,
                  size_t workspace_bytes, void* stream);

/* pk_w4a16_gemm with a bias in the epilogue: C[m, n] = tensor_scale * (A @ dequant(B))[m, n]
 * + bias[n], rounded once to the output dtype, where bias is N values of bias_dtype (PK_F32,
 * PK_F16 or PK_BF16; null: none). Every kernel pk_w4a16_gemm runs adds it where it stores
 * the output (its own epilogue, the split-K handoff or the reduce launch). Same plan,
 * workspace and errors as pk_w4a16_gemm. Replaces the linear layer's `x @ w.T + b` of the
 * reference's quantized model (quantize.py:160-181 writes w back into nn.Linear, whose
 * forward adds the layer's bias). */
int pk_w4a16_gemm_bias(const void* a, int64_t lda, const uint32_t* qweight, int64_t ldq,
                       const void* scales, int group_size, float tensor_scale, const void* bias,
                       int bias_dtype, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                       int split_k, void* workspace, size_t workspace_bytes, void* stream);

/* pk_w4a16_gemm_bias on weights stored in blocks: the same codes as pk_w4a16_gemm's (K, N/8)
 * words, reordered into blocks of 128 rows x 256 columns (16 KB, row-major inside), the
 * blocks ordered by row block and then column tile -- word j of row k at
 * ((k / 128) * (N / 256) + j / 32) * 4096 + (k % 128) * 32 + j % 32, i.e. torch's
 * qweight.view(K/128, 128, N/256, 32).permute(0, 2, 1, 3). A workgroup then streams 16 KB
 * runs instead of one 128-byte line per 5.5 KB row, while the column tiles that a GEMM works
 * on at the same k stay adjacent (measured on MI355X: the M=1 4096x11008 GEMV 4% faster,
 * Llama-3-8B layers at M = 1..32 up to 12%, the large GEMMs within 2%). Same scales, bias,
 * output, split_k, plan, workspace (pk_w4a16_workspace_bytes) and bits as pk_w4a16_gemm_bias
 * with ldq = N/8. Requires N % 256 == 0, K % 256 == 0, group_size % 64 == 0 with scales,
 * 16-byte aligned operands, and a plan on a kernel that reads blocks (M <= 4, the
 * register-dequant kernel, or the packed-B GEMM; the automatic split always is): otherwise
 * PK_EUNSUPPORTED. Has no counterpart in the reference, whose int4 weights exist only in
 * pack_int4_n order (gemm_int4.py:65-72); it is the layout QuantLinear keeps in memory (its
 * file format stays pack_int4_n order). */
int pk_w4a16_gemm_tiled(const void* a, int64_t lda, const uint32_t* qtiled, const void* scales,
                        int group_size, float tensor_scale, const void* bias, int bias_dtype,
                        void* c, int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                        void* workspace, size_t workspace_bytes, void* stream);

/* W4A16 decode matmul (1 <= M <= 8) on weights in the strip layout: C = tensor_scale * A @
 * dequant(q, S) (+ bias), the arithmetic of pk_w4a16_gemm_bias (gemm_int4.py:21-55, 75-92 with
 * group scales), in ONE launch with no split-K partials: one workgroup per 16-column strip
 * (or per two: pk_w4a16_strips_plan) adds the whole of K in LDS, in a fixed order (bitwise
 * reproducible). The strip layout is a
 * byte permutation of pack_int4_n's (K, N/2) bytes (gemm_int4.py:65-72): byte (k, c), with
 * k = 128b + 32rs + 8g + e and c = 8s + 2cps + h (b block, rs, g, cps in 0..3, e in 0..7,
 * h in 0..1), sits at byte ((((s * K/128 + b) * 4 + g) * 4 + rs) * 4 + cps) * 16 + 8h + e, both
 * nibbles XOR 8 (the code biased to 0..15): each strip's K rows contiguous, in 1 KB blocks of
 * 128 rows. Scales (group mode, sstrips non-null):
 * the (K/G, N) fp16 group scales reordered as (N/16, K/G, 16). Requires N % 16 == 0,
 * K % 128 == 0, G a multiple of 32 dividing K that divides 128 or is a multiple of it,
 * 16-byte aligned A rows and weights, 8-byte aligned scales; fp32/fp16/bf16 output and bias.
 * Replaces gemm_int4.int4_gemm (gemm_int4.py:75-92) at 1 <= M <= 8 and the split-K GEMV
 * (gemm_splitk.py:26-80) for decode: the reference has no weight layout other than
 * pack_int4_n's. */
int pk_w4a16_gemm_strips(const void* a, int64_t lda, const uint8_t* qstrips, const void* sstrips,
                         int group_size, float tensor_scale, const void* bias, int bias_dtype,
                         void* c, int c_dtype, int64_t ldc, int M, int N, int K, void* stream);

/* Fix the strip GEMV's 1 KB blocks per wave (2, 4 or 8) for later calls, or 0 for the
 * automatic choice; for measurements. No counterpart in the reference. */
int pk_w4a16_strips_config(int blocks_per_wave);

/* The launch pk_w4a16_gemm_strips plans for M rows of an (N, K) layer: 16-column strips per
 * workgroup (1, or 2 for 2..8 rows on layers with strips enough: each wave then multiplies
 * the same blocks of two strips by one load of their activations), 1 KB blocks per wave per
 * round, and waves per workgroup (any output pointer may be NULL). For tests and measurement;
 * no counterpart in the reference. */
int pk_w4a16_strips_plan(int M, int N, int K, int* strips_per_workgroup, int* blocks_per_wave,
                         int* waves);

/* pk_w4a16_gemm_strips bound to one set of strip-layout weights, for eager decode loops that
 * pay host time per call: pk_w4a16_strips_prepare checks the fixed arguments (weights, scales,
 * group, tensor scale, bias, output dtype, N, K and the activations' row stride lda) and plans
 * M = 1..8 once; pk_w4a16_strips_run then takes only the activations, the output and its row
 * stride, the row count and the stream, and launches the same kernel with the same bits. The
 * handle holds pointers, not copies: the weights, scales and bias must stay allocated and in
 * place until pk_w4a16_strips_release. prepare returns NULL on a bad argument
 * (pk_last_error says which); run returns PK_OK or an error code. A handle is read-only after
 * prepare, so runs on several streams may share it. No counterpart in the reference (a
 * Triton launch has no prepared form). */
void* pk_w4a16_strips_prepare(const uint8_t* qstrips, const void* sstrips, int group_size,
                              float tensor_scale, const void* bias, int bias_dtype, int c_dtype,
                              int N, int K, int64_t lda);
int pk_w4a16_strips_run(void* prepared, const void* a, void* c, int64_t ldc, int M, void* stream);
void pk_w4a16_strips_release(void* prepared);

/* pk_w4a16_strips_run with timing: the dispatch itself records start_event (a hipEvent_t) as
 * the kernel starts and stop_event as it ends (either may be NULL; both must exist already),
 * so a run of calls can be timed from its first kernel's start to its last kernel's end with
 * no event packet of its own between them. Same launch, same bits. For measurement; no
 * counterpart in the reference. */
int pk_w4a16_strips_run_events(void* prepared, const void* a, void* c, int64_t ldc, int M,
                               void* stream, void* start_event, void* stop_event);

/* Rows per kernel call of pk_w4a16_gemm_tiled for M activation rows of stride lda elements:
 * M itself while the activations span less than 2 GiB (M * lda * 2 bytes); beyond that the
 * call runs equal chunks of this many rows (a multiple of 128), since the kernels that read
 * block-layout weights at large M address their operands with 32-bit buffer offsets; 0 when
 * even 128 rows exceed that. No device work. No counterpart in the reference (a Triton launch
 * addresses its operands with 64-bit pointers). */
int64_t pk_w4a16_tiled_rows_per_call(int64_t M, int64_t lda);

/* Which kernel pk_w4a16_gemm would run and its split factor (for reporting/benchmarks):
 * writes kernel id (1 = GEMV for M <= 4, 2 = LDS-tiled MFMA GEMM that dequantises B into LDS,
 * 3 = register-dequant MFMA kernel for 5 <= M <= 64, and M <= 128 on layers of at most
 * 4096 x 4096 weights: with an automatic split where the layer has at least 1024 x 1024
 * weights and the kernel's plan needs at most 8 slices, else where the next kernel does not
 * take the shape, 4 = MFMA GEMM that keeps B packed in
 * LDS, for M > 64, and with an automatic split for M > 32 on layers of more than 4096 x 8192
 * weights, with N % 256 == 0, K % 128 == 0, group % 64 == 0 (split-K with a reduce
 * launch where its tiles leave CUs idle), assuming 16-byte aligned operands) and the
 * effective split. */
int pk_w4a16_plan(int M, int N, int K, int group_size, int split_k, int* kernel_id,
                  int* split_used);

/* Kernel launches pk_w4a16_gemm makes for this shape on the current device: 1, or 2 when
 * split-K partials are added by a separate pk_splitk_reduce launch (negative on error).
 * Assumes aligned operands (the GEMV's MFMA path); for benchmarks and reporting. No
 * counterpart in the reference (its split-K is one Triton launch plus atomics). */
int pk_w4a16_launches(int M, int N, int K, int group_size, int split_k);

/* Activations for a packed layer of the reference's quantize_model layout (one fp32 scale per
 * input feature over all output rows: quantize.py:52-54 through rtn_layer / gptq_layer with
 * group_size=None, written back at quantize.py:179): y[m, k] = fp16(x[m, k] * in_scale[k] *
 * mul) for x (M, K) fp32 / fp16 / bf16 with row stride ldx, y fp16 with 16-byte aligned rows
 * (ldy % 8 == 0), K % 8 == 0. The layer's product x @ wq^T is then pk_w4a16_gemm of y with
 * the int4 codes, no group scales and tensor_scale = 1 / mul. in_scale NULL: the input cast
 * alone. Replaces the dequantisation q * s of quantize_col (quantize.py:54) by the same scale
 * on the activation side. */
int pk_w4a16_prep_activations(const void* x, int x_dtype, int64_t ldx, const float* in_scale,
                              float mul, void* y, int64_t ldy, int M, int K, void* stream);

/* Fixes the register-dequant kernel's (kernel id 3) layout for every later plan in the
 * process: 8 or 16 output columns per lane and 4 or 8 waves per workgroup; (0, 0) restores
 * the automatic choice. Layouts with the same wave count give the same bits; the wave count
 * changes the fp32 summation order only. For layout tests and tuning; the environment
 * variable PK_SKINNY_CFG="cols,waves" sets the same once, at the first plan. Not thread-safe
 * against concurrent plans in the sense that a call in flight may use either layout. No
 * counterpart in the reference. PK_EINVAL for other values. */
int pk_w4a16_skinny_layout(int cols_per_lane, int waves);

/* pk_w4a16_gemm for callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc): no workspace argument, and the call allocates nothing. No
 * counterpart in the reference. The split-K workspace is a fixed device array inside the
 * library, pk_w4a16_noalloc_scratch_bytes() bytes (16 MiB) per GPU, held until the process
 * ends; shapes whose plan needs more return PK_EWORKSPACE (pk_w4a16_workspace_bytes() gives
 * the need). The first call on a device looks the array up and clears its counters on
 * `stream`; every call leaves them zero. Every call on a GPU shares that GPU's array: calls
 * that overlap in time on one GPU (different streams, threads) race and must not be made.
 * Results are bitwise those of pk_w4a16_gemm with the same arguments. */
size_t pk_w4a16_noalloc_scratch_bytes(void);
int pk_w4a16_gemm_noalloc(const void* a, int64_t lda, const uint32_t* qweight, int64_t ldq,
                          const void* scales, int group_size, float tensor_scale, void* c,
                          int c_dtype, int64_t ldc, int M, int N, int K, int split_k,
                          void* stream);

/* The two phases of a split-K pk_w4a16_gemm, for callers that reduce elsewhere (for example
 * across devices) or time the phases separately. pk_w4a16_gemm_partials writes the fp32
 * partial sums of every slice to `partials`, laid out (split, M, N) -- the per-slice products
 * of gemm_splitk.gemm_splitk_kernel (gemm_splitk.py:26-61) before its atomic add -- and
 * pk_splitk_reduce forms C = scale * sum over slices in slice order 0..split-1, the ordered
 * replacement of that atomic add (gemm_splitk.py:64). `split` must be the effective split of
 * pk_w4a16_plan (>= 2); partials_bytes >= split * M * N * 4. */
int pk_w4a16_gemm_partials(const void* a, int64_t lda, const uint32_t* qweight, int64_t ldq,
                           const void* scales, int group_size, float* partials,
                           size_t partials_bytes, int M, int N, int K, int split_k,
                           void* stream);
int pk_splitk_reduce(const float* partials, int split, int M, int N, float scale, void* c,
                     int c_dtype, int64_t ldc, void* stream);

/* ------------------------------------------------------------------------------------- */
/* Dense fp16 matmul with deterministic split-K                                          */
/* ------------------------------------------------------------------------------------- */

/* C[M,N] (fp32/fp16) = A[M,K] (fp16) @ B[K,N] (fp16, row-major, row stride ldb), fp32
 * accumulate, K split into split_k contiguous slices reduced in fixed order.
 * Requires K % (32 * split_k) == 0 and N % 8 == 0.
 * Replaces gemm_splitk.triton_gemm_splitk (gemm_splitk.py:67-80) and, with split_k = 1,
 * gemm.triton_gemm (gemm.py:103-128); the reference reduces split-K slices with fp32
 * atomics, this reduction is ordered and reproducible. */
size_t pk_gemm_f16_workspace_bytes(int M, int N, int K, int split_k);
int pk_gemm_f16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int c_dtype,
                int64_t ldc, int M, int N, int K, int split_k, void* workspace,
                size_t workspace_bytes, void* stream);

/* pk_gemm_f16 with bf16 A and B (bf16 MFMA, fp32 accumulate); the same constraints and
 * workspace (pk_gemm_f16_workspace_bytes). Replaces gemm.triton_gemm (gemm.py:103-128) for
 * bf16 and gemm_splitk.triton_gemm_splitk (gemm_splitk.py:67-80) with bf16 inputs; the
 * reference serves both dtypes from one tl.dot. */
int pk_gemm_bf16(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int c_dtype,
                 int64_t ldc, int M, int N, int K, int split_k, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------- */
/* fp8 e4m3 matmul                                                                       */
/* ------------------------------------------------------------------------------------- */

/* C[M,N] = out_scale * (A8[M,K] @ B8[K,N]) with e4m3 inputs, fp32 accumulation and the
 * scale applied once in the epilogue; C is fp32/fp16/bf16.
 * b_layout 0: B8 is (K, N) row-major with row stride ldb (the reference layout);
 * b_layout 1: B8 is stored transposed, (N, K) row-major with row stride ldb.
 * Requires K % 16 == 0, M, N >= 1, 16-byte aligned rows (the reference's mask-free kernel
 * needs K to be a multiple of its autotuned BLOCK_K, 32 or 64).
 * Replaces gemm_fp8.fp8_gemm_precast / fp8_gemm_kernel (gemm_fp8.py:38-86, 98-117). */
int pk_fp8_gemm(const uint8_t* a8, int64_t lda, const uint8_t* b8, int64_t ldb, int b_layout,
                float out_scale, void* c, int c_dtype, int64_t ldc, int M, int N, int K,
                void* stream);

/* ------------------------------------------------------------------------------------- */
/* GPTQ column sweep                                                                     */
/* ------------------------------------------------------------------------------------- */

/* Quantizes columns [b0, b0 + nb) of q (fp32 [out, ldq], GPTQ column order) one after another,
 * in place: column c's value is q[:, c] minus, in column order, err[:, j] * ratio[j][c] for
 * the block's earlier columns j (each product rounded before its subtraction), then it is
 * RTN-quantized with `bits` (qmax = 2^(bits-1) - 1) and one scale per `group` consecutive rows
 * (group 0: one scale per column): s = max|v|.clamp_min(1e-12) / qmax, q = clamp(rint(v/s),
 * -qmax, qmax) * s. err (fp32 [out, lde]) receives v - q at column c - b0. ratio is fp32
 * [in, ldr] with ratio[j][c] = Hinv[j, c] / Hinv[j, j]. Updates from columns before b0 must
 * already be applied to q (the caller's GEMM). nb <= pk_gptq_block_cols(out, group).
 * Replaces the inner loop of quantize.gptq_layer (quantize.py:104-110). */
int pk_gptq_block_cols(int out, int group);
int pk_gptq_block(float* q, int64_t ldq, const float* ratio, int64_t ldr, float* err, int64_t lde,
                  int out, int in, int b0, int nb, int bits, int group, void* stream);

/* ------------------------------------------------------------------------------------- */
/* Split-KV decode attention                                                             */
/* ------------------------------------------------------------------------------------- */

/* Single-query attention per (batch b, head h) over N cached keys/values:
 *   out[b,h,:] = softmax(q . K^T * sm_scale) @ V   (fp32 out, (B, H, D) contiguous),
 * computed FlashDecoding-style: K/V split into N/split slices of `split` rows, per-slice
 * (max, sum, acc) partials in fp32, then one combine in slice order (bitwise reproducible).
 * q is (B, H, D) fp16 with strides sqb, sqh; k and v are (B, H, N, D) fp16 with strides
 * (skb, skh, skn) / (svb, svh, svn) and unit stride along D (a KV-cache prefix view is read
 * in place). D in {16, 32, 64, 128, 256}; any split with N % split == 0 (the reference's
 * Triton kernel takes powers of two); 16-byte aligned rows.
 * workspace: pk_flash_decode_workspace_bytes() bytes, zero-filled once before its first use
 * (its first 64 KiB are the arrival counters, shared with pk_w4a16_gemm: every call leaves
 * them zero again), so one workspace per stream serves both.
 * pk_flash_decode_launches: 1 when the slices are combined inside the split kernel (B*H <=
 * 512 on an XCD count of 1, 2, 4 or 8), else 2 (a combine kernel follows); 0 for a bad shape.
 * Replaces flash_decoding.flash_decoding (flash_decoding.py:84-115) and its kernel
 * flash_decoding_kernel (:48-81). */
size_t pk_flash_decode_workspace_bytes(int B, int H, int N, int D, int split);
int pk_flash_decode_launches(int B, int H, int N, int D, int split);
int pk_flash_decode(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb,
                    int64_t skh, int64_t skn, const void* v, int64_t svb, int64_t svh,
                    int64_t svn, int B, int H, int N, int D, int split, float sm_scale,
                    float* out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PICO_KERNELS_AMD_H */
