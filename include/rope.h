/* rope: rotary position embedding (rotate-half / NeoX pairing, full rotary) of q[tokens, q_heads, head_dim] and
 * k[tokens, kv_heads, head_dim] in bf16 (qk_dtype 1) or fp16 (2). Library: build/rope/libkernel.so. Replaces the
 * reference's rope/kernel.cu:201-215 (ctypes binding rope/candidate.py:28). Device pointers, row-major contiguous;
 * asynchronous on `stream`; no allocation. q_out may equal q and k_out may equal k (in-place rotation). Return: 0
 * success (tokens <= 0 is a no-op), -1 invalid argument (tokens > 2^31 - 1, head_dim odd or <= 0, q_heads or kv_heads
 * <= 0, rows < 1, splits outside [1, 65535], unsupported dtype), otherwise the hipError_t of the launch. */
#ifndef ROWKERN_ROPE_H
#define ROWKERN_ROPE_H
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

/* rope/kernel.cu:201: cos_rows/sin_rows are a cache [P, head_dim] in fp32 (cache_dtype 0), bf16 (1) or fp16 (2), ids
 * the int64 position of each token (a row of the cache, in [0, P)). `rows` and `splits` are the reference's CUDA
 * block-shape hints: validated as there, otherwise unused. */
int launch(const void* q, const void* k, const void* cos_rows, const void* sin_rows, const void* ids, void* q_out,
           void* k_out, long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype, int cache_dtype,
           int rows, int splits, hipStream_t stream);

/* No counterpart in the reference (which reads a cache): cos/sin computed on the fly, cos = fp32(cos(t)) and
 * sin = fp32(sin(t)) of t = fp32(float(pos) * inv_freq[i]) for inv_freq[head_dim / 2] (fp32, device memory), the same
 * pair at i and i + head_dim / 2 -- equal to a cache built from inv_freq with fp32 angles. Same shapes, in-place rule
 * and codes as launch(); inv_freq == NULL is -1. */
int rope_launch_freq(const void* q, const void* k, const void* ids, const float* inv_freq, void* q_out, void* k_out,
                     long long tokens, int q_heads, int kv_heads, int head_dim, int qk_dtype, hipStream_t stream);

/* No counterpart in the reference (the step after RoPE in a decoder layer): RoPE fused with the KV-cache write.
 * q_out = rope(q) with cos/sin on the fly as rope_launch_freq (q_out may equal q); the rotated k and the unrotated v
 * of token t go to row slot_mapping[t] (int64) of k_cache and v_cache, each [slots, kv_heads, head_dim] in
 * the qk dtype -- a paged [blocks, block_size, kv_heads, head_dim] cache with slot = block * block_size + offset; a
 * negative slot writes nothing for its token. k and v are only read. Same checks and codes as rope_launch_freq; a null
 * v, cache or slot_mapping is -1. */
int rope_kv_launch(const void* q, const void* k, const void* v, const void* ids, const float* inv_freq, void* q_out,
                   void* k_cache, void* v_cache, const void* slot_mapping, long long tokens, int q_heads, int kv_heads,
                   int head_dim, int qk_dtype, hipStream_t stream);

/* No counterpart in the reference: tuning override for parameter sweeps. Slots: 0 threads per block, 1 resident blocks
 * per CU, 2 forced scalar kernel (1). Returns 0 or -1. */
int rope_tune(int slot, int value);

#ifdef __cplusplus
}
#endif
#endif
