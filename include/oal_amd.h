/*
 * oal_amd.h -- C ABI of the MI355X (gfx950) OAL grouped quadratic attention library.
 *
 * One shared library, liboal_amd.so, built with hipcc for gfx950. Every entry point
 * takes plain device pointers and sizes; no framework types cross this boundary.
 * Callers own every buffer (inputs, outputs, the forward's saved state and the
 * backward's workspace; sizes come from the *_bytes queries). Work is enqueued on
 * the caller's HIP stream and nothing is synchronized (oal_backward, and
 * oal_forward on the fp32 route, may run part of their work on a second stream
 * of the library's own, forked from and joined back to the caller's stream by
 * events, so the caller sees one stream). The library allocates no device
 * memory.
 *
 * Operator (reference oal_attention/grouped_reference.py:102-211):
 *   s_g(i,j)   = scale * sum_{d: labels[h][d] == g} q[i][d] * k[j][d]
 *   kappa(i,j) = c0[h] + sum_g lam[h][g] s_g + sum_{g,g'} gam[h][g][g'] s_g s_g'
 *   num[i] = sum_{j<=i} kappa(i,j) v[j],  den[i] = sum_{j<=i} kappa(i,j)
 *   out[i] = num[i] / max(den[i], floor)        (floor <= 0: plain num / den)
 * gam must be symmetric. The head dimension and value dimension are 64 (callers
 * with smaller dimensions pad q, k, v with zeros). Query head h reads KV head
 * h / (q_heads / kv_heads).
 *
 * Layouts (row-major, contiguous):
 *   q [B][Hq][N][64], k and v [B][Hkv][N][64]    dtype OAL_DTYPE_F32 or OAL_DTYPE_BF16
 *   out [B][Hq][N][64] (dtype);  num [B][Hq][N][64] f32;  den [B][Hq][N] f32
 *   labels [Hq][64] int32 in [0, groups);  c0 [Hq];  lam [Hq][groups];
 *   gam [Hq][groups][groups]  (all f32);  1 <= groups <= 64
 * The q, k, v, out, num, den, saved, workspace, dout, dnum, dden, dq, dk and dv
 * pointers must be 16-byte aligned (the kernels move rows with 16-byte accesses);
 * a misaligned one is rejected with an error, before anything is enqueued.
 *
 * Return value: 0 on success, nonzero on invalid arguments or a launch error;
 * oal_last_error() then describes the failure (thread-local string).
 */
#ifndef OAL_AMD_H_
#define OAL_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OAL_DTYPE_F32 0
#define OAL_DTYPE_BF16 1

/* Arithmetic precision (reference HD planner "precision", hd_block_gemm.py:132-153):
 * OAL_PRECISION_FP32  fp32 arithmetic throughout (VALU kernels), any group count.
 * OAL_PRECISION_BF16  bf16 operands, fp32 accumulation on the gfx950 matrix cores
 *                     (MFMA) for any group count up to 64 and up to 8 query heads
 *                     per KV head (more run the fp32 kernels). Up to 8 groups the
 *                     intra-chunk term is formed from group sums; more groups --
 *                     per-pair coefficients, labels d -> d with 64 groups -- form
 *                     the intra-chunk local score in feature form,
 *                     phi_Q . phi_K^T on the matrix cores. */
#define OAL_PRECISION_FP32 0
#define OAL_PRECISION_BF16 1

/* ABI revision of this header. */
int oal_abi_version(void);

/* Message for the last nonzero return on the calling thread. */
const char* oal_last_error(void);

/* Opt-in per-kernel timing. While enabled, every kernel launch is bracketed by
 * HIP events recorded on the launch stream. oal_profile_collect() waits for the
 * recorded events, writes one line "kernel_name launches total_ms" per kernel
 * into buf (NUL-terminated, truncated to buflen) and clears the records. This
 * replaces the reference's CUDA-event stage timing
 * (oal_attention/hd_block_gemm_profiling.py:195-226). */
int oal_profile_enable(int enable);
int oal_profile_collect(char* buf, size_t buflen);

/* Logical feature count 1 + 64 + 64*65/2 = 2145 (reference
 * hd_block_gemm_cache.py:105-121 pair layout) and the padded stride used in
 * the saved state. */
int oal_feature_count(void);
int oal_feature_stride(void);

/* Token block (chunk) the kernels use; results do not depend on it. */
int oal_chunk_size(void);

/* Bytes of the forward's saved state (per-chunk exclusive prefix states and
 * feature coefficients), needed by oal_backward. */
size_t oal_forward_saved_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups, int dtype,
                               int precision);

/* Bytes of scratch oal_backward needs. */
size_t oal_backward_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups, int dtype,
                                    int precision);

/*
 * Causal chunked forward. Replaces the forward of the reference's HD Block-GEMM
 * core, oal_attention/hd_block_gemm_runtime.py:617-805 (_hd_parallel_block_gemm_impl,
 * called through hd_block_gemm_autograd.py:85-204), and of the legacy Triton
 * route oal_attention/triton/grouped_quadratic_causal_forward_kernels.py:1155-1386.
 * Writes out, num, den and the saved state.
 */
int oal_forward(const void* q, const void* k, const void* v,
                const int32_t* labels, const float* c0, const float* lam, const float* gam,
                int groups, int batch, int q_heads, int kv_heads, int seq_len, int dtype,
                int precision, float scale, float floor,
                void* out, float* num, float* den, void* saved, void* stream);

/*
 * First-order VJP. Replaces oal_attention/hd_block_gemm_autograd.py:207-347
 * (_hd_parallel_block_gemm_autograd_backward_impl) and the legacy
 * grouped_causal_first_order_vjp (triton/grouped_quadratic_causal_backward.py:1807-1869).
 * dout (dtype), dnum [B][Hq][N][64] f32 and dden [B][Hq][N] f32 may each be NULL
 * (no upstream gradient). dq, dk, dv (dtype) and the coefficient gradients
 * dc0 [Hq], dlam [Hq][groups], dgam [Hq][groups][groups] (f32, overwritten) may be
 * NULL when not requested; dc0, dlam and dgam are requested together (all or
 * none), and on the bf16 path dk and dv are too. dgam is the gradient of
 * sum_{g,g'} gam[g][g'] s_g s_g' with gam a symmetric matrix: an off-diagonal
 * entry carries the mean of the two routings of its pairs. (The reference's
 * gather, grouped_reference.py:89-93, routes pair (r, c), r >= c, to
 * [g(r)][g(c)] only; gradients reaching a factor L with gam = L L^T, or a
 * per-pair coefficient, are the same under both.) Invalid combinations are
 * refused before anything is enqueued. On the matrix-core paths (bf16, and fp32
 * with up to 8 groups) most of the intra-chunk VJP and of the query-side fold
 * run on a second stream, on the bf16 group-sum path at up to 128 chunks per
 * unit with the denominator kernels (one per device, default
 * priority, created with its fork/join events on the first call; not created
 * while the caller's stream is capturing a graph, whose call then stays on the
 * caller's stream). Every kernel on it waits for an event recorded on the
 * caller's stream, and at the end of the call the caller's stream waits for the
 * last of them, so work enqueued after the call, or an event recorded after it,
 * covers all of it.
 */
int oal_backward(const void* q, const void* k, const void* v,
                 const int32_t* labels, const float* c0, const float* lam, const float* gam,
                 int groups, int batch, int q_heads, int kv_heads, int seq_len, int dtype,
                 int precision, float scale, float floor,
                 const float* num, const float* den, const void* saved,
                 const void* dout, const float* dnum, const float* dden,
                 void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam,
                 void* workspace, void* stream);

/*
 * Allocation-free variant of oal_backward. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as oal_backward, without the workspace: the workspace
 * is a file-scope device array of OAL_NOALLOC_SCRATCH_BYTES (256 MiB) that each
 * GPU the library runs on holds until the process ends, whether or not this
 * entry point is called (the array is part of the loaded code object). It runs
 * all its kernels on the caller's stream (no second stream). A geometry whose
 * oal_backward_workspace_bytes exceeds it is refused with an error (B = 1,
 * N = 4096, 14/2 heads needs 146 MiB on the bf16 path). Nothing is allocated or
 * freed. The stream must belong to the current device. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two host
 * threads) race and must be serialized by the caller.
 */
#define OAL_NOALLOC_SCRATCH_BYTES (256u << 20)
int oal_backward_noalloc(const void* q, const void* k, const void* v,
                         const int32_t* labels, const float* c0, const float* lam, const float* gam,
                         int groups, int batch, int q_heads, int kv_heads, int seq_len, int dtype,
                         int precision, float scale, float floor,
                         const float* num, const float* den, const void* saved,
                         const void* dout, const float* dnum, const float* dden,
                         void* dq, void* dk, void* dv, float* dc0, float* dlam, float* dgam,
                         void* stream);

/*
 * Matrix-core self-test: one wave checks the MFMA accumulator layouts and the
 * transposed LDS read (ds_read_b64_tr_b16) lane mapping the bf16 kernels
 * assume, and adds the number of mismatching elements to
 * *device_errors (a device int the caller zeroed). No counterpart in the
 * reference; it lets a deployment verify the device before trusting results.
 */
int oal_selftest(int* device_errors, void* stream);

/*
 * FP64 evaluation, the route of oal_attention(execution="reference") when the
 * working dtype is float64. Replaces the reference's float64 evaluation of
 * grouped_quadratic_reference (oal_attention/grouped_quadratic.py:332-355,
 * grouped_reference.py:102-211) and, for the backward, torch autograd of it.
 * Same operator and layouts as oal_forward with every tensor float64: q, k, v
 * (padded to 64 features), c0 [Hq], lam [Hq][groups], gam [Hq][groups][groups]
 * (symmetric), out and num [B][Hq][N][64], den [B][Hq][N]; out = num / den, no
 * floor. Evaluated over token pairs in 32-token tiles (O(N^2) per head), for
 * validation in double precision rather than speed. No saved state: the
 * backward recomputes from q, k, v.
 */
int oal_forward_f64(const double* q, const double* k, const double* v,
                    const int32_t* labels, const double* c0, const double* lam, const double* gam,
                    int groups, int batch, int q_heads, int kv_heads, int seq_len, double scale,
                    double* out, double* num, double* den, void* stream);

/* Workspace of oal_backward_f64 in bytes (0 on invalid geometry). */
size_t oal_backward_f64_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int groups);

/*
 * VJP of oal_forward_f64, every tensor float64: dout [B][Hq][N][64], dnum
 * [B][Hq][N][64] and dden [B][Hq][N] may each be NULL; dq, dk, dv, and the
 * coefficient gradients dc0, dlam, dgam (requested together) may be NULL when
 * not requested. dgam is in the symmetric convention of oal_backward.
 */
int oal_backward_f64(const double* q, const double* k, const double* v,
                     const int32_t* labels, const double* c0, const double* lam, const double* gam,
                     int groups, int batch, int q_heads, int kv_heads, int seq_len, double scale,
                     const double* num, const double* den,
                     const double* dout, const double* dnum, const double* dden,
                     double* dq, double* dk, double* dv, double* dc0, double* dlam, double* dgam,
                     void* workspace, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OAL_AMD_H_ */
