/* topk: the k largest entries of each row of x[rows, cols] in fp32 (dtype 0) or bf16 (dtype 1), sorted descending with
 * ties broken by the lowest index (+0 above -0, +NaN above +inf, -NaN at the bottom: the composite order of the
 * reference), 1 <= k <= 1024. Library: build/topk/libkernel.so. Replaces the reference's topk/kernel.cu:520-570 (ctypes
 * binding topk/candidate.py:31-36). Device pointers; asynchronous on `stream`. As in the reference, the caller owns
 * the workspace and the counters (topk/candidate.py:38-63) and the library allocates nothing and keeps no device
 * state: a split row's chunks hand their results over in the caller's work and count their arrivals on the caller's
 * counters[row]. */
#ifndef ROWKERN_TOPK_H
#define ROWKERN_TOPK_H
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

/* topk/kernel.cu:520: columns per workgroup for a rows x cols launch (the row's chunk count is ceil(cols / chunk)),
 * sized so the grid is resident about once; a chunk longer than one 16384-element register tile is rounded up to whole
 * tiles, never shorter than min_chunk, a multiple of 8 when a row is split. `threads` and `depth` are the reference's
 * CUDA tuning knobs, accepted and unused. */
long long plan(long long rows, long long cols, int dtype, int threads, int depth, int min_chunk);

/* topk/kernel.cu:549: values [rows, k] in x's dtype, indices [rows, k] int64; work: u64 [rows * nchunks * k]
 * (nchunks = ceil(cols / chunk)), the chunk results of split rows; counters: u32 [>= rows], zero on entry and left
 * zero (a split row's last chunk to arrive merges, as in the reference, and zeroes counters[row]). The launch may join
 * chunks into fewer, longer ones, which stays inside that work: for k <= 64 a last chunk too short to give each of
 * a workgroup's four waves a 16-byte vector is folded into the previous chunk when the two fit one 16384-element
 * register tile; for k > 64 a row is split into at most min(256, k) chunks of at least 16k columns (the result does
 * not depend on the chunking). For k > 64 the chunks also leave their bounds in the row's indices before the merge
 * writes them.
 * Returns 0 (rows <= 0 or k <= 0 is a no-op), -1 for k > cols, k > 1024, cols > INT_MAX / 2, rows > 65535, chunk <= 0,
 * a split row with chunk % 4 != 0 or nchunks * k > INT_MAX / 2, threads not 128/256/512, depth not 2/4/8, an unknown
 * dtype or (this build's addition) a split row with a null work or counters, otherwise the hipError_t of the launch.
 * Launches sharing work/counters must be ordered (one stream). */
int launch(const void* x, void* values, void* indices, void* work, void* counters, long long rows, long long cols,
           int k, int dtype, int threads, int depth, long long chunk, hipStream_t stream);

/* No counterpart in the reference: launch() for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The same arguments and checks without work and
 * counters, which live in a static scratch of the library, one per GPU, held until the process ends: 256 KiB of row
 * counters and 16 MiB of chunk results. Each call zeroes its counters with a small kernel first (no memset node) and
 * allocates nothing. -1 also when a split row's results would not fit: rows * nchunks * k u64 slots (rows * nchunks
 * for k = 1) above 16 MiB, counted over the chunks the launch runs (k > 64 lengthens chunks shorter than 16k columns,
 * k <= 64 may fold a short last chunk into the one before). All calls on one GPU share that GPU's scratch: calls that
 * overlap on one GPU (two streams, two host threads) race and must be ordered by the caller. */
int topk_launch_noalloc(const void* x, void* values, void* indices, long long rows, long long cols, int k, int dtype,
                        int threads, int depth, long long chunk, hipStream_t stream);

/* No counterpart in the reference (whose counters self-reset only when a launch completes): zeroes counters[0, rows)
 * on `stream` with a small kernel, for a caller recovering from a launch that did not complete. Returns 0, -1 (NULL
 * counters) or the hipError_t of the launch. */
int topk_reset(void* counters, long long rows, hipStream_t stream);

/* No counterpart in the reference (the step after top-k in a decoder's sampler): one index per row drawn
 * from a top-k list -- values [rows, k] in fp32 (dtype 0) or bf16 (1) and int64 indices [rows, k], as launch() writes
 * them -- with the caller's uniforms[rows] (fp32 in [0, 1)). x = value / temperature, e_i = exp(x_i - max x),
 * S_i = e_0 + ... + e_i; the positions i with i == 0 or S_(i-1) < top_p * S_(k-1) are kept, and the first kept i with
 * S_i > u * S_(last kept) is drawn. temperature <= 0 is greedy (position 0); top_p >= 1 keeps every position. Values
 * must be finite when temperature > 0. out: int64 [rows]. Returns 0 (rows <= 0 is a no-op), -1 for k outside
 * [1, 1024], rows > 2^31 - 1, a null pointer or an unknown dtype, otherwise the hipError_t of the launch. */
int topk_sample_launch(const void* values, const void* indices, const float* uniforms, void* out, long long rows, int k,
                       int dtype, float temperature, float top_p, hipStream_t stream);

/* No counterpart in the reference (the top-k launch of a decoder's sampler, with the draw fused in): launch() plus, in
 * the same kernel, topk_sample_launch()'s draw from each row's list -- the workgroup that writes a row's values and
 * indices draws out[row] from them, so out equals topk_sample_launch() on launch()'s output and one launch (and its
 * launch gap) is saved. Arguments and checks of launch(), plus uniforms[rows] (fp32 in [0, 1)), out (int64 [rows]),
 * temperature (<= 0: greedy) and top_p (>= 1: no nucleus cut); -1 also for a null uniforms or out when rows > 0. */
int topk_launch_sample(const void* x, void* values, void* indices, void* work, void* counters, long long rows,
                       long long cols, int k, int dtype, int threads, int depth, long long chunk, const float* uniforms,
                       void* out, float temperature, float top_p, hipStream_t stream);

/* No counterpart in the reference: tuning override for parameter sweeps. Slot 0: resident workgroups per CU assumed by
 * plan(); slot 1: 1 makes launch() take the naive tier (one workgroup per row, one scan of the row per output
 * position: the harness's seed column). Returns 0 or -1. */
int topk_tune(int slot, int value);

#ifdef __cplusplus
}
#endif
#endif
