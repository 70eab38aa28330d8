/*
 * pk_bench_probes.h -- measurement probes for bench.py (libpk_bench_probes.so). Not part of
 * the product library or its C ABI (include/pico_kernels_amd.h); no counterpart in the
 * reference. The probes return 0, -1 for a bad argument, or the HIP error code of the launch.
 */
#ifndef PK_BENCH_PROBES_H
#define PK_BENCH_PROBES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Launches `grid` workgroups of 8 waves that each issue iters x 8 independent MFMAs (fp8 != 0:
 * v_mfma 32x32x64 e4m3, else 32x32x16 fp16) on constant (random == 0) or pseudo-random register
 * operands, with no memory traffic in the loop; out receives grid * 512 floats. FLOPs per
 * launch: grid * 8 * iters * 8 * (fp8 ? 131072 : 32768). */
int pkb_mfma_probe(int fp8, int random, int grid, int iters, float* out, void* stream);

/* Reads `bytes` (a multiple of 16, 16-byte aligned) with `grid` workgroups of 256 threads and
 * writes one 32-bit word per workgroup (the XOR of the words it read) to out. */
int pkb_read_probe(const void* src, size_t bytes, uint32_t* out, int grid, void* stream);

/* The strip GEMV's read pattern alone: one workgroup of 8 waves per strip of strip_bytes
 * (a multiple of 1024, below 2 GiB) contiguous bytes at src (16-byte aligned), each wave
 * loading u (1, 2, 4 or 8) consecutive 1 KB blocks per round; out receives 8 words per
 * workgroup (8 * 8 * ceil(strips / 8) in all). */
int pkb_strip_read_probe(const void* src, int strips, int64_t strip_bytes, int u, uint32_t* out,
                         void* stream);

/* The partition's XCD count (hipDeviceAttributeNumberOfXccs of the current device), or -1. */
int pkb_xcc_count(void);

/* Launches `grid` workgroups of `threads` threads (a multiple of 64, at most 1024) holding
 * `lds_bytes` (4..65536) of LDS; each sleeps about spin * 64 clocks (0..100000) and writes the
 * XCC id it ran on to out[workgroup]. */
int pkb_xcc_probe(int grid, int threads, int lds_bytes, int spin, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PK_BENCH_PROBES_H */
