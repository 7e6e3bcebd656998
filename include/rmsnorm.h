/* rmsnorm: y = x * inv over the last dim of x[rows, cols], inv = rsqrt(mean(x^2) + eps) rounded to x's dtype, for bf16
 * (dtype 1) and fp16 (dtype 2). Library: build/rmsnorm/libkernel.so. Replaces the reference's rmsnorm/kernel.cu:132-139
 * (ctypes binding rmsnorm/candidate.py:26-28). Device pointers, row-major contiguous; asynchronous on `stream`; no
 * allocation. Return: 0 success (rows <= 0 is a no-op), -1 invalid argument (rows > 2^31 - 1, cols <= 0, threads not a
 * multiple of 32 in [32, 1024], unsupported dtype), otherwise the hipError_t of the launch. */
#ifndef ROWKERN_RMSNORM_H
#define ROWKERN_RMSNORM_H
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

/* rmsnorm/kernel.cu:132. `threads` is the reference's CUDA block size: validated as there, otherwise unused. */
int launch(const void* x, void* y, long long rows, int cols, int dtype, float eps, int threads, hipStream_t stream);

/* No counterpart in the reference (which has no weight): y = T(weight * T(x * inv)) with weight[cols] in x's dtype,
 * torch's `weight * y` on dtype tensors. weight == NULL gives launch()'s result. Same checks and codes as launch(). */
int rmsnorm_launch_weighted(const void* x, const void* weight, void* y, long long rows, int cols, int dtype,
                            float eps, int threads, hipStream_t stream);

/* No counterpart in the reference (the step before an inference layer's norm): fused residual add.
 * h = T(x + residual) is written to residual_out, then y = RMSNorm(h), times weight when weight != NULL, in one pass
 * (x and residual read once, residual_out and y written once). residual_out may equal residual and y may equal x.
 * Same checks and codes as launch(); residual or residual_out NULL is -1. */
int rmsnorm_add_launch(const void* x, const void* residual, const void* weight, void* y, void* residual_out,
                       long long rows, int cols, int dtype, float eps, int threads, hipStream_t stream);

/* No counterpart in the reference: tuning override for parameter sweeps. Slots: 0 waves per row, 1 vectors per lane,
 * 2 resident blocks per CU, 3 forced generic kernel (1), 4 non-temporal loads (default on; 2 off). Returns 0 or -1. */
int rmsnorm_tune(int slot, int value);

#ifdef __cplusplus
}
#endif
#endif
