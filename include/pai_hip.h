/*
 * pai_hip — MI355X (gfx950) quantized-weights matmul behind ProsperoAI's
 * C operator interface.
 *
 * Computes y[M][N] = x[M][K] · Wᵀ where W[N][K] is stored as GGUF blocks
 * (Q8_0, Q4_0, Q4_K, Q6_K) in the native GGUF row layout, x and y are f32
 * row-major. This is the GPU twin of the reference's per-projection CPU
 * operator, which is the composition
 *     pai_gguf_dequant     (adapters/llama/gguf.c:969-1012, blocks → f32)
 *   → transpose2d          (adapters/llama/llama.c:196-209, [N][K] → [K][N])
 *   → pai_ref_gemm_f32     (cpu/reference/ref_ops.c:427-444)
 * called from the executor's run_gemm (scheduler/scheduler.c:285-343).
 *
 * ABI conventions follow cpu/optimized/opt_ops.h:36-81 and
 * cpu/reference/ref_ops.h: free C functions, uint64_t dimensions, raw
 * pointers, pai_status_t returns; PAI_ERR_INVALID_ARG for NULL pointers or
 * zero dimensions; the caller owns x and y. No call aborts the process:
 * HIP failures map to PAI_ERR_INIT / NOMEM / INTERNAL / TIMEOUT.
 *
 * Thread-safety: init/shutdown are idempotent and serialised internally.
 * Calls on different pai_qmat_t handles may run concurrently; calls on
 * one handle must not overlap (the handle owns the MFMA path's activation
 * workspace). The synchronous entry points run on the default stream and
 * wait for it; their host-pointer staging buffer is shared under a lock.
 */
#ifndef PAI_HIP_H
#define PAI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: same type and values as sdk/include/pai/error.h:11-23, so a
 * caller that already includes <pai/error.h> sees identical definitions. */
typedef int32_t pai_status_t;
#ifndef PAI_OK
#define PAI_OK 0
#define PAI_ERR_INVALID_ARG -1
#define PAI_ERR_NOMEM -2
#define PAI_ERR_UNSUPPORTED -3
#define PAI_ERR_CAPABILITY -4
#define PAI_ERR_TIMEOUT -5
#define PAI_ERR_MISMATCH -6
#define PAI_ERR_IO -7
#define PAI_ERR_INIT -8
#define PAI_ERR_INTERNAL -9
#define PAI_ERR_PROTOCOL -10
#endif

/* Block formats accepted by pai_qmat_upload. The values are the ggml type
 * ids used in GGUF files (adapters/llama/gguf.h:34-51: Q4_0 = 2, Q8_0 = 8,
 * Q4_K = 12, Q6_K = 14); other ids return PAI_ERR_UNSUPPORTED. */
#define PAI_QTYPE_Q4_0 2u
#define PAI_QTYPE_Q8_0 8u
#define PAI_QTYPE_Q4_K 12u
#define PAI_QTYPE_Q6_K 14u

/* ---------------------------------------------------------------------- */
/* Lifecycle                                                               */
/* ---------------------------------------------------------------------- */

/* Select the current HIP device, check it is gfx950 and load the kernels.
 * Idempotent; PAI_ERR_INIT when no usable device is present.
 * Replaces nothing in the reference (its runtime has no GPU bring-up on
 * this path; runtime/runtime.c:17-81 is the CPU analogue). */
pai_status_t pai_hip_init(void);

/* Release the host-pointer staging buffer. Idempotent. Handles stay valid
 * until their pai_qmat_free (which also frees their workspace). */
pai_status_t pai_hip_shutdown(void);

/* Human-readable text of the last failure on this thread ("" if none). */
const char *pai_hip_last_error(void);

/* Launch-shape overrides for measurements and tests. All knobs start at 0,
 * which is the shipped dispatch; nothing reads the environment. Not
 * thread-safe against concurrent compute calls (set them before enqueuing).
 * No counterpart in the reference. INVALID_ARG for an unknown knob or a
 * negative value; out-of-range values are ignored by the dispatch. */
#define PAI_TUNE_GEMM_SPLITS 1u        /* MFMA GEMM K parts, 1..64            */
#define PAI_TUNE_GEMM_NO_X16 2u        /* 1: MFMA path without the 16-bit copy */
#define PAI_TUNE_GEMM_ATOMIC_SPLITS 3u /* 1: multi-matrix parts via atomics   */
#define PAI_TUNE_GEMV_WGS 4u           /* GEMV workgroups                     */
#define PAI_TUNE_GEMV_ROWS 5u          /* GEMV rows per group: 1, 2 or 4      */
#define PAI_TUNE_GEMV_NW 6u            /* one-token GEMV waves: 8 or 16       */
#define PAI_TUNE_GEMV_NO_MX 7u         /* 1: no matrix-core GEMV for 2..8 tokens */
#define PAI_TUNE_MFMA_MIN_M 8u         /* tokens from which the MFMA GEMM runs */
#define PAI_TUNE_GEMM_TILE 9u          /* 16-bit GEMM token tile: 1, 2, 3 = 32, 128, 256 */
#define PAI_TUNE_V0_SEQUENTIAL 10u     /* 1: v0 GEMMs one thread per output  */
pai_status_t pai_hip_set_tuning(uint32_t knob, int32_t value);

/* Bytes occupied by `numel` elements of `type`; 0 when numel is not a
 * whole number of blocks or the type is not one of the four above.
 * Same semantics as pai_gguf_type_bytes (adapters/llama/gguf.c:562-597)
 * restricted to those types. */
uint64_t pai_qtype_bytes(uint32_t type, uint64_t numel);

/* ---------------------------------------------------------------------- */
/* Packed weights resident in HBM                                          */
/* ---------------------------------------------------------------------- */

typedef struct pai_qmat pai_qmat_t;

/* Copy W[N][K] in native GGUF block layout (N rows of K/blk blocks, the
 * bytes pai_gguf_dequant reads at adapters/llama/gguf.c:1003) from host
 * memory into device memory, re-laid out for the kernels. Dequantized
 * values are unchanged, bit for bit.
 * Replaces the session-init load (models/model.c:242-298) for GGUF-tagged
 * weights: the blocks are uploaded instead of being dequantized into the
 * host region.
 * Errors: INVALID_ARG (NULL, zero dims), UNSUPPORTED (type, or K not a
 * whole number of blocks), MISMATCH (nbytes != N * pai_qtype_bytes(K)),
 * NOMEM (device allocation), INIT (no device). */
pai_status_t pai_qmat_upload(pai_qmat_t **out, uint32_t type, uint64_t n,
                             uint64_t k, const void *blocks, uint64_t nbytes);

/* Same, from native blocks already in device memory (`stream` is a
 * hipStream_t or NULL for the calling thread's stream; the call returns
 * after the re-layout completes). */
pai_status_t pai_qmat_upload_device(pai_qmat_t **out, uint32_t type,
                                    uint64_t n, uint64_t k,
                                    const void *dev_blocks, uint64_t nbytes,
                                    void *stream);

/* Free the device copy. NULL is a no-op returning PAI_OK. */
pai_status_t pai_qmat_free(pai_qmat_t *w);

/* Type and shape of a handle. */
pai_status_t pai_qmat_shape(const pai_qmat_t *w, uint32_t *type, uint64_t *n,
                            uint64_t *k);

/* Packed bytes of the matrix (N * pai_qtype_bytes(K)); 0 for NULL. */
uint64_t pai_qmat_bytes(const pai_qmat_t *w);

/* ---------------------------------------------------------------------- */
/* GGUF files: tensor directory and upload without dequantization          */
/* ---------------------------------------------------------------------- */

/* Read-only tensor directory over a GGUF file held in memory (for example
 * mmap'ed). It does not own the buffer, which must outlive it. */
typedef struct pai_gguf_dir pai_gguf_dir_t;

/* Parse the header, metadata and tensor infos. Accepts exactly the files
 * pai_gguf_open accepts (adapters/llama/gguf.h:76-78, gguf.c:128-245) with
 * the same codes: PROTOCOL for malformed input (short file, bad magic,
 * reads past the end, unknown metadata type, empty or >= 128-byte names,
 * n_dims outside 1..4, extents above 2^26, a bad alignment, a data section
 * past the end), UNSUPPORTED for versions outside 1..3 or more than 1024
 * tensors; NOMEM, INVALID_ARG for NULL. Metadata values are skipped, except
 * "general.alignment". */
pai_status_t pai_gguf_dir_open(const void *data, uint64_t size,
                               pai_gguf_dir_t **out);

/* Free the directory (not the buffer). NULL is a no-op. */
void pai_gguf_dir_close(pai_gguf_dir_t *d);

/* Number of tensors (pai_gguf_t.tensor_count); 0 for NULL. */
uint64_t pai_gguf_dir_count(const pai_gguf_dir_t *d);

/* File version, alignment and byte offset of the data section from the
 * start of the buffer (pai_gguf_t.version / .alignment / .data_start).
 * Any output may be NULL. */
pai_status_t pai_gguf_dir_layout(const pai_gguf_dir_t *d, uint32_t *version,
                                 uint32_t *alignment, uint64_t *data_start);

/* Tensor info `index` (0-based, file order): the fields of
 * pai_gguf_tensor_t (adapters/llama/gguf.h:54-60). `name` stays valid until
 * pai_gguf_dir_close; dims receives 4 extents, innermost first, unused ones
 * 0; offset is relative to the data section. Any output may be NULL.
 * INVALID_ARG for an index out of range. */
pai_status_t pai_gguf_dir_tensor(const pai_gguf_dir_t *d, uint64_t index,
                                 const char **name, uint32_t *type,
                                 uint32_t *n_dims, uint64_t *dims,
                                 uint64_t *offset);

/* Index of the first tensor named exactly `name`; MISMATCH when absent
 * (pai_gguf_find_tensor, adapters/llama/gguf.h:98-99, returns NULL). */
pai_status_t pai_gguf_dir_find(const pai_gguf_dir_t *d, const char *name,
                               uint64_t *index);

/* Pointer into the buffer at tensor `index`'s native blocks and their byte
 * count, after the checks pai_gguf_dequant makes before reading them
 * (adapters/llama/gguf.c:984-996): PROTOCOL for zero elements or bytes
 * outside the file, UNSUPPORTED for a type other than the four block
 * formats or an element count that is not whole blocks. */
pai_status_t pai_gguf_dir_blocks(const pai_gguf_dir_t *d, uint64_t index,
                                 const void **blocks, uint64_t *nbytes);

/* Upload the 2-D tensor `name` (extents [K, N], innermost first) as a
 * resident matrix W[N][K], straight from its native blocks: no dequant, no
 * transpose. Replaces, for GPU sessions, the per-tensor import in
 * adapters/llama/llama.c:408-470 (pai_gguf_find_tensor, pai_gguf_dequant,
 * transpose2d). Errors: MISMATCH (absent, or not 2-D), then those of
 * pai_gguf_dir_blocks and pai_qmat_upload. */
pai_status_t pai_qmat_upload_gguf(pai_qmat_t **out, const pai_gguf_dir_t *d,
                                  const char *name);

/* ---------------------------------------------------------------------- */
/* Compute                                                                  */
/* ---------------------------------------------------------------------- */

/* flags for pai_qgemm_f32 / pai_qdequant_f32 */
#define PAI_QGEMM_DEVICE_PTRS (1u << 0) /* x, y (out) are device pointers  */
#define PAI_QGEMM_MFMA_BF16 (1u << 1)   /* 16-bit MFMA path: bf16 operands  */
#define PAI_QGEMM_FP32 (1u << 2)        /* any M: f32 dequant + f32 FMA path */

/* y[m][n] = sum_k x[m][k] * W[n][k], x: [M][K] f32, y: [M][N] f32.
 *  - M < 8, M = 8 when K is a multiple of 128 up to 4096, or
 *    PAI_QGEMM_FP32: blocks are multiplied with exact integer dot products
 *    against a 24-bit image of x and f32 accumulation (one token on the
 *    vector ALUs, 2 to 8 tokens per launch on the i8 matrix cores where K
 *    is a multiple of 128). Matches the reference's sequential f32 sum
 *    within rel-L2 1e-5.
 *  - Otherwise (the 16-bit MFMA path): blocks are dequantized in registers to fp16 (default) or
 *    bf16, x is rounded to the same type, and MFMA accumulates in f32.
 *    Tolerance: rel-L2 <= 2e-3 (fp16), <= 1.6e-2 (bf16). fp16 operands
 *    need |x| < 65504 (larger values become inf); bf16 has the f32 range.
 *    Each matrix keeps a device workspace for a 16-bit copy of up to 1024
 *    tokens of x, allocated by the first such call made outside stream
 *    capture; calls of up to 32 tokens round x inside the GEMM instead
 *    and use no copy (same rounding, same bits). Workspaces only grow: a buffer replaced by a larger one stays
 *    allocated until pai_qmat_free, because a HIP graph captured earlier
 *    still refers to it. Destroy every graph that used a handle before
 *    freeing the handle.
 *    Repeatability: results repeat bit for bit, except where a
 *    single-matrix launch whose tiles do not fill the chip splits K into
 *    more than two parts (e.g. 4096 rows at 40 or 512 tokens, 4096 x 14336
 *    at 8 to 512 tokens): its parts are added with f32 atomics in arrival
 *    order, and the sums differ between calls in the last bits, within the
 *    tolerance above. Multi-matrix calls sum their parts in a fixed order.
 * Without PAI_QGEMM_DEVICE_PTRS, x and y are host pointers and the call
 * copies them; with it, they are device pointers. Synchronous.
 * Replaces pai_ref_gemm_f32 at scheduler/scheduler.c:340 for a weight
 * value carrying the GGUF tag, i.e. the composition described above. */
pai_status_t pai_qgemm_f32(const pai_qmat_t *w, uint64_t m, const float *x,
                           float *y, uint32_t flags);

/* Asynchronous form: x and y must be device pointers; `stream` is a
 * hipStream_t (NULL = the default stream). Returns once the kernels are
 * enqueued; argument and shape errors are reported before any launch. */
pai_status_t pai_qgemm_f32_async(const pai_qmat_t *w, uint64_t m,
                                 const float *x, float *y, uint32_t flags,
                                 void *stream);

/* pai_qgemm_f32_async that allocates nothing: no hipMalloc, hipFree or
 * other allocating call, on any path. On the 16-bit MFMA path the 16-bit
 * copy of x lives in a 16 MiB device array of the library (one per GPU,
 * held until the process ends) instead of the handle's workspace, in token
 * blocks that fit it; the GEMV paths need no scratch. Same arguments,
 * errors and numerics as pai_qgemm_f32_async; results are bit-identical to
 * it wherever that call's launches repeat bit for bit and both run the
 * tokens as one block (up to 16 MiB / (2 K) tokens, rounded down to a
 * multiple of 256, and at most 1024). PAI_ERR_UNSUPPORTED when the MFMA
 * path would need K > 32768 (256 tokens of 16-bit activations must fit).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race; serialise them on one stream.
 * No counterpart in the reference. It exists for callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, and
 * harnesses that forbid device allocation. */
pai_status_t pai_qgemm_f32_noalloc_async(const pai_qmat_t *w, uint64_t m,
                                         const float *x, float *y,
                                         uint32_t flags, void *stream);

/* Fused projections: y_i[m][N_i] = x[m][K] * W_i^T for `count` (1..4)
 * matrices that share the activations (the q/k/v or gate/up projections
 * of one layer). All matrices must have the same type and K (otherwise
 * PAI_ERR_MISMATCH). x and every y_i are device pointers; `stream` is a
 * hipStream_t (NULL = the default stream); the call returns once the
 * kernels are enqueued. On the integer-dot path (see pai_qgemm_f32) the
 * matrices are multiplied in one launch per token group, which streams all
 * of their blocks and converts x once; results are bit-identical to
 * separate pai_qgemm_f32_async calls. On the 16-bit MFMA path the matrices
 * share one launch, whose K split is chosen for all of them together and
 * whose parts are summed in a fixed order: results are within the MFMA
 * tolerance of separate calls, and bit-identical to them when neither
 * splits K.
 * No counterpart in the reference, whose executor runs each projection as
 * its own pai_ref_gemm_f32 (scheduler/scheduler.c:340); this is the fused
 * form of those calls for weights that share an input value
 * (adapters/llama/llama.c:678-696, :760-772). */
pai_status_t pai_qgemm_f32_multi_async(const pai_qmat_t *const *ws, uint32_t count,
                                       uint64_t m, const float *x, float *const *ys,
                                       uint32_t flags, void *stream);

/* Feed-forward gate/up with its activation fused:
 *   h[m][N] = silu(x W_gate^T) * (x W_up^T),  silu(g) = g / (1 + e^-g).
 * Replaces the reference's four ops GEMM(gate), GEMM(up), SILU, MUL
 * (adapters/llama/llama.c:760-784, executed at scheduler/scheduler.c:340,
 * :484-488, :404-410); the gate and up products are never written out.
 * W_gate and W_up must have the same type, N and K (PAI_ERR_MISMATCH).
 * x and h are device pointers; `stream` as for pai_qgemm_f32_async.
 *  - On the integer-dot path (see pai_qgemm_f32): one launch per token
 *    group streams both matrices and applies the epilogue; the gate and up
 *    sums are those pai_qgemm_f32_async computes for the same tokens, bit
 *    for bit, and silu uses the device expf (within 4 ulp of the
 *    reference's f32 composition applied to them). One token, or K not a
 *    multiple of 128: K up to 18720 (PAI_ERR_UNSUPPORTED above).
 *  - Otherwise: the gate product is written to h, then the up product's
 *    epilogue replaces each element by silu(h) * up (that launch is not
 *    split over K). Tolerances of the MFMA path. */
pai_status_t pai_qgemm_f32_gate_up_async(const pai_qmat_t *w_gate,
                                         const pai_qmat_t *w_up, uint64_t m,
                                         const float *x, float *h,
                                         uint32_t flags, void *stream);

/* out[N][K] = dequantized W in the native element order, computed on the
 * GPU from the device copy; bit-identical to pai_gguf_dequant
 * (adapters/llama/gguf.c:650-967) for every value, with one exception: a
 * block whose f16 scale is a NaN gives a quiet NaN, where the reference
 * keeps the scale's payload bits (gguf.c:620-621). Every other f16 scale
 * pattern, subnormals and infinities included, converts identically. Host
 * pointer unless PAI_QGEMM_DEVICE_PTRS. Synchronous. */
pai_status_t pai_qdequant_f32(const pai_qmat_t *w, float *out, uint32_t flags);

/* ---------------------------------------------------------------------- */
/* The executor's GEMM branch                                               */
/* ---------------------------------------------------------------------- */

/* run_gemm's shape rules (scheduler/scheduler.c:280-338) for a GGUF
 * weight of w_n rows of w_k columns, whose graph value has the logical
 * shape [w_k][w_n]. Shapes are (rank, dims) of the op's values a, b, c:
 *   is_gemv: y[m] = A[m,k] x[k] with A the weight: a = [w_n, w_k],
 *            b = [k], c = [m]; m = w_n, n = 1 output per row;
 *   a of rank 1 (row vector): y[n] = x[k] W[k,n]: b = [w_k, w_n],
 *            c = [n] or [1, n]; m = 1;
 *   otherwise C[m,n] = A[m,k] W[k,n]: a = [m, k], b = [w_k, w_n],
 *            c = [m, n].
 * Writes the product's tokens (*m_tokens: rows of activations) and
 * returns MISMATCH where run_gemm does (rank or extent mismatch), and
 * also when the weight side differs from the weight's own shape;
 * INVALID_ARG for NULL shape arrays or out pointers. Host-only; no
 * counterpart beyond run_gemm's own checks. */
pai_status_t pai_qgemm_shape_check(int is_gemv, uint32_t a_rank, const uint64_t *a_shape,
                                   uint32_t b_rank, const uint64_t *b_shape, uint32_t c_rank,
                                   const uint64_t *c_shape, uint64_t w_n, uint64_t w_k,
                                   uint64_t *m_tokens);

/* The GEMM/GEMV branch itself for a GGUF-tagged weight: the shape check
 * above against w's shape, then pai_qgemm_f32 on the activations `act`
 * (the operand that is not the weight: b for the GEMV form, a
 * otherwise) into `out` (c), with `flags` as pai_qgemm_f32 (host
 * pointers, or device pointers with PAI_QGEMM_DEVICE_PTRS). Replaces the
 * pai_ref_gemm_f32 call of scheduler/scheduler.c:340 for such a weight. */
pai_status_t pai_qgemm_run(const pai_qmat_t *w, int is_gemv, uint32_t a_rank,
                           const uint64_t *a_shape, uint32_t b_rank, const uint64_t *b_shape,
                           uint32_t c_rank, const uint64_t *c_shape, const float *act,
                           float *out, uint32_t flags);

/* ---------------------------------------------------------------------- */
/* CPU reference twin                                                       */
/* ---------------------------------------------------------------------- */

/* y[m][n] = x[m][k] * W^T on the host, W[N][K] given as native GGUF blocks
 * (`blocks`, N rows of K/blk blocks) of `type`: the reference's CPU
 * composition for such a weight, pai_gguf_dequant (adapters/llama/
 * gguf.c:650-947) then pai_ref_gemm_f32 on the transposed values
 * (cpu/reference/ref_ops.c:427-444), bit for bit. Argument order follows
 * pai_ref_gemm_f32 (m, n, k, a, b, c) with the format first. This is the
 * ref_fn of the qgemm_* descriptors (PAI_OP_CAP_CPU_REF), which the
 * reference's executor requires of every op it schedules
 * (scheduler/scheduler.c:749-756); no GPU entry point calls it, and it
 * allocates nothing. Errors: INVALID_ARG (NULL, zero dims), UNSUPPORTED
 * (type, or K not a whole number of blocks). */
pai_status_t pai_qgemm_ref_f32(uint32_t type, uint64_t m, uint64_t n,
                               uint64_t k, const float *x, const void *blocks,
                               float *y);

/* ---------------------------------------------------------------------- */
/* v0 per-group formats (models/quantize.h)                                 */
/* ---------------------------------------------------------------------- */

/* Same field order, types and size as pai_quant_scheme_t
 * (models/quantize.h:36-40): bit_width 4 or 8, is_signed 1, group_size 0
 * for one group over the whole array. */
typedef struct pai_hip_quant_scheme {
  uint8_t bit_width;
  uint8_t is_signed;
  uint16_t group_size;
} pai_hip_quant_scheme_t;

/* c[m][n] = a[m][k] * W, W[k][n] stored as the reference's quantized-GEMM
 * operands (cpu/reference/ref_ops.h:154-183): w_q int8 codes at t*n+j
 * (w8), or two 4-bit codes per byte over that flat index (w4: low nibble
 * for even indices, sign-extended), with one f32 scale per (group of
 * group_size rows, column) at b_scales[(t/group_size)*n + j]; group_size 0
 * or > k is one group over k. Same signatures and error codes as
 * pai_ref_gemm_w8_f32 / pai_ref_gemm_w4_f32 (ref_ops.c:446-499), which
 * they replace; host pointers, synchronous (the operands are copied to the
 * device and back on every call, so they suit a registry dispatch with
 * host buffers; resident weights use pai_hip_gemm_wq_f32_async).
 * Results are within the f32 tolerance of the reference's sequential sum
 * (rel-L2 1e-5 and below); shapes whose n is not a multiple of 16, or
 * whose group_size is neither a multiple of 16 nor >= k, take a kernel
 * that reproduces the reference's sum bit for bit. Dimensions up to
 * 2^31 - 1 (UNSUPPORTED above). */
pai_status_t pai_hip_gemm_w8_f32(uint64_t m, uint64_t n, uint64_t k,
                                 const float *a, const int8_t *w_q,
                                 const float *b_scales, uint64_t group_size,
                                 float *c);
pai_status_t pai_hip_gemm_w4_f32(uint64_t m, uint64_t n, uint64_t k,
                                 const float *a, const int8_t *w_q4,
                                 const float *b_scales, uint64_t group_size,
                                 float *c);

/* The same product on device pointers, enqueued on `stream` (a
 * hipStream_t; NULL = default stream); bits 8 or 4. `workspace` (device
 * memory, may be NULL) holds the split-K parts of small-M calls, which
 * are summed in a fixed order by a second launch, so results repeat bit
 * for bit; PAI_HIP_WQ_WORKSPACE_BYTES is enough for every shape, and a
 * smaller or NULL workspace only reduces the split. Nothing is allocated.
 * Calls sharing a workspace must not overlap. */
#define PAI_HIP_WQ_WORKSPACE_BYTES (4u << 20)
pai_status_t pai_hip_gemm_wq_f32_async(uint32_t bits, uint64_t m, uint64_t n,
                                       uint64_t k, const float *a,
                                       const void *w_q, const float *b_scales,
                                       uint64_t group_size, float *c,
                                       void *workspace,
                                       uint64_t workspace_bytes, void *stream);

/* models/quantize.h:63-75 on the GPU, bit for bit: per group
 * scale = max|x| / qmax (127 or 7; NaN elements do not count),
 * q = lrintf(x / scale) clamped to +-qmax (0 for a zero scale), 4-bit
 * codes two per byte with element 2i in the low nibble (an odd tail's
 * high nibble 0); out = scale * q. Same signatures and errors as
 * pai_quantize_f32 / pai_dequantize_f32 (models/quantize.c:74-181): host
 * pointers, synchronous. n up to 2^31 - 1 (UNSUPPORTED above). */
pai_status_t pai_hip_quantize_f32(const float *src, uint64_t n,
                                  const pai_hip_quant_scheme_t *scheme,
                                  int8_t *out_q, float *out_scales,
                                  uint64_t *out_num_groups);
pai_status_t pai_hip_dequantize_f32(const int8_t *q, const float *scales,
                                    uint64_t n,
                                    const pai_hip_quant_scheme_t *scheme,
                                    float *out);
/* Device-pointer forms on `stream`: out_q and out 16-byte aligned. The
 * session's load of a v0 tensor (models/model.c:264-290) maps to one
 * pai_hip_dequantize_f32_async into the device region. */
pai_status_t pai_hip_quantize_f32_async(const float *src, uint64_t n,
                                        const pai_hip_quant_scheme_t *scheme,
                                        int8_t *out_q, float *out_scales,
                                        uint64_t *out_num_groups, void *stream);
pai_status_t pai_hip_dequantize_f32_async(const int8_t *q, const float *scales,
                                          uint64_t n,
                                          const pai_hip_quant_scheme_t *scheme,
                                          float *out, void *stream);

/* CPU twins of pai_ref_gemm_w8_f32 / pai_ref_gemm_w4_f32 (the same
 * signatures and results, bit for bit): the ref_fn of the qgemm_w8_f32 /
 * qgemm_w4_f32 descriptors. They allocate nothing. */
pai_status_t pai_gemm_w8_ref_f32(uint64_t m, uint64_t n, uint64_t k,
                                 const float *a, const int8_t *w_q,
                                 const float *b_scales, uint64_t group_size,
                                 float *c);
pai_status_t pai_gemm_w4_ref_f32(uint64_t m, uint64_t n, uint64_t k,
                                 const float *a, const int8_t *w_q4,
                                 const float *b_scales, uint64_t group_size,
                                 float *c);

/* ---------------------------------------------------------------------- */
/* IR quantization tag of GGUF block weights                                */
/* ---------------------------------------------------------------------- */

/* The block structure a GGUF-tagged IR value carries: one more value of
 * pai_ir_quant_block_t (ir/ir.h:88-93), after PAI_IR_QUANT_BLOCK_GROUP,
 * so PAI_IR_QUANT_BLOCK_COUNT becomes 4 and pai_ir_value_set_quant
 * (ir/ir.c:62-80) accepts it unchanged otherwise. */
#define PAI_IR_QUANT_BLOCK_GGUF 3u

/* Same field order, types and size as pai_ir_quant_t (ir/ir.h:95-103); the
 * repr fields hold pai_ir_quant_repr_t values (0 = F32, 1 = F16). */
typedef struct pai_hip_ir_quant {
  uint8_t present;
  uint8_t bit_width;
  uint8_t scale_repr;
  uint8_t zero_point_repr;
  uint8_t is_signed;
  uint8_t block_structure;
  uint16_t group_size;
} pai_hip_ir_quant_t;

/* The tag of a block format: block_structure PAI_IR_QUANT_BLOCK_GGUF and
 *   Q8_0  8 bits, signed,   group 32,  f16 scale
 *   Q4_0  4 bits, unsigned, group 32,  f16 scale (codes offset by 8)
 *   Q4_K  4 bits, unsigned, group 256, f16 scale, f16 min (zero-point repr)
 *   Q6_K  6 bits, signed,   group 256, f16 scale (int8 sub-scales)
 * (bit_width, group_size, is_signed) tells the four apart. UNSUPPORTED for
 * other types, INVALID_ARG for NULL. No counterpart in the reference,
 * whose importer dequantizes GGUF weights instead of tagging them
 * (adapters/llama/llama.c:408-470). */
pai_status_t pai_hip_quant_tag(uint32_t type, pai_hip_ir_quant_t *out);

/* The ggml type id a tag denotes (PAI_QTYPE_*), or 0 when the tag is NULL,
 * absent, not GGUF-structured, or none of the four formats. */
uint32_t pai_hip_quant_type(const pai_hip_ir_quant_t *q);

/* ---------------------------------------------------------------------- */
/* Op-registry descriptors                                                  */
/* ---------------------------------------------------------------------- */

/* Capability bit for ops with a HIP implementation on gfx950. The
 * reference defines bits 0-2 (sdk/include/pai/op.h:59-61). */
#define PAI_OP_CAP_GPU_HIP (1u << 3)

/* Same field order, types and size as pai_op_descriptor_t
 * (sdk/include/pai/op.h:71-82), so a pointer to one of these can be
 * passed to pai_op_registry_register (runtime/op_registry.c) unchanged.
 * The dtype fields hold pai_dtype_t values (sdk/include/pai/dtype.h:12-23;
 * 0 = PAI_DTYPE_F32, 8 = PAI_DTYPE_U8). */
typedef struct pai_hip_op_descriptor {
  const char *name;
  uint32_t version;
  uint32_t num_inputs;
  uint32_t num_outputs;
  int32_t in_dtype;
  int32_t out_dtype;
  uint32_t caps;
  pai_status_t (*ref_fn)(void);
  int32_t kernel_id;
  uint32_t reserved[2];
} pai_hip_op_descriptor_t;

/* Six descriptors. "qgemm_q4_0_f32", "qgemm_q8_0_f32", "qgemm_q4_k_f32",
 * "qgemm_q6_k_f32": inputs x f32 and the packed weight, output y f32,
 * ref_fn pai_qgemm_ref_f32. "qgemm_w8_f32", "qgemm_w4_f32": inputs a,
 * w_q, b_scales as the builtin gemm_w8_f32 / gemm_w4_f32
 * (runtime/op_registry.c:268-285), ref_fn pai_gemm_w8_ref_f32 /
 * pai_gemm_w4_ref_f32. All carry caps PAI_OP_CAP_CPU_REF |
 * PAI_OP_CAP_GPU_HIP and kernel_id PAI_KERNEL_NONE; the dispatch site
 * casts ref_fn to the prototype, as it casts the builtins' ref_fn. The
 * array is static and outlives any registry it is registered into. */
const pai_hip_op_descriptor_t *pai_hip_op_descriptors(uint32_t *count);

/* Registry name for a ggml type ("qgemm_q4_k_f32"), NULL if unsupported. */
const char *pai_hip_op_name(uint32_t type);

#ifdef __cplusplus
}
#endif

#endif /* PAI_HIP_H */
