/* softmax: row-wise softmax over the last dim, fp32 (dtype 0) and bf16 (dtype 1) rows, fp32 accumulation.
 * Library: build/softmax/libkernel.so. Replaces the reference's softmax/kernel.cu:520-527 (and the same ABI of
 * softmax/seed.cu:68-81). x and y are device pointers to row-major contiguous [rows, cols] data; the call is
 * asynchronous on `stream` and allocates nothing except, for rows longer than 32768 fp32 / 65536 bf16 elements, small
 * per-(device, stream) workspaces the library keeps (chunk pairs; for the single-pass tier also per-row counters, which
 * every launch leaves at zero). Launches sharing a stream are ordered by it. Return: 0 success (rows <= 0 or cols <= 0
 * is a no-op), -1 unsupported dtype, otherwise the hipError_t of the launch. */
#ifndef ROWKERN_SOFTMAX_H
#define ROWKERN_SOFTMAX_H
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

/* softmax/kernel.cu:520. `threads` and `aux` are the reference's block-size hints for its CUDA tiers; accepted and not
 * used (the tier and shape are chosen from the row length). */
int launch(const void* x, void* y, long long rows, long long cols, int dtype, int threads, int aux,
           hipStream_t stream);

/* No counterpart in the reference: tuning override for parameter sweeps (slot, value; 0 restores the automatic
 * choice). Slots: 0 waves per row, 1 vectors per lane, 2 resident blocks per CU, 3 split-tier waves, 4 split-tier
 * vectors per lane, 5 forced tier (1 row, 2 split, 3 generic, 4 co-resident), 6 non-temporal loads (1 on). Returns 0
 * or -1. */
int softmax_tune(int slot, int value);

#ifdef __cplusplus
}
#endif
#endif
