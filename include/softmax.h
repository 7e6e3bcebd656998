/* softmax: row-wise softmax over the last dim, fp32 (dtype 0) and bf16 (dtype 1) rows, fp32 accumulation.
 * Library: build/softmax/libkernel.so. Replaces the reference's softmax/kernel.cu:520-527 (and the same ABI of
 * softmax/seed.cu:68-81). x and y are device pointers to row-major contiguous [rows, cols] data; the call is
 * asynchronous on `stream` and allocates nothing. Rows longer than 32768 fp32 / 65536 bf16 elements whose chunks fit
 * on the GPU at once are done in one pass by co-resident workgroups that exchange their chunk statistics through a
 * static device table of the library (entries tagged per launch, nothing to clear); launches on one stream are ordered
 * by it, and a launch overlapping another on a second stream stays exact (at worst its workgroups stop waiting after
 * about 100 us and read their row again). Graph capture: a call on a capturing stream records a one-wave kernel node
 * ahead of the softmax kernel node, which gives every replay fresh tags on the device, so replays of a captured launch
 * are exact on whatever x holds at replay time; no memset node is recorded. Each captured co-resident launch keeps one
 * of 4096 tag cells per device for the life of the process; once they are used up, further captured launches of such
 * rows take the two-pass stream tier. Return: 0 success (rows <= 0 or cols <= 0 is a no-op), -1 unsupported dtype,
 * otherwise the hipError_t of the launch. */
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

/* No counterpart in the reference: tuning override for parameter sweeps and tests (slot, value; 0 restores the
 * automatic choice). Slots: 0 waves per row, 1 vectors per lane, 2 resident blocks per CU, 3 stream-tier waves, 4
 * co-resident row groups, 5 preferred tier (1 row, 2 stream, 3 generic, 4 co-resident; a tier that cannot take the
 * rows is passed over), 6 non-temporal loads (1 on), 7 the co-resident wait budget in 100 MHz ticks. Returns 0 or -1. */
int softmax_tune(int slot, int value);

#ifdef __cplusplus
}
#endif
#endif
