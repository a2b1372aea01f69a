/*
 * mxq.h — C ABI of libmxq: the MLX affine group-quantized linear on MI355X
 * (gfx950), written from scratch in HIP.
 *
 * Each entry point replaces one operation that the reference reaches through
 * MLX-Swift (third-party mlx-swift 0.32.3, which wraps the mlx-c C API):
 *
 *   mxq_quantize          <- quantized(w, groupSize:, bits:)
 *                            `model/minimax h3/tools/quantize_h3_g64.py:132`,
 *                            `Packages/z-image-swift/Sources/ZImage/Weights.swift:31`
 *   mxq_dequantize        <- dequantized(wq, scales:, biases:, groupSize:, bits:)
 *                            `model/minimax h3/H3Common.swift:382-401`
 *   mxq_quantized_matmul  <- quantizedMM / quantizedMatmul(x, w, scales:, biases:,
 *                            transpose: true, groupSize:, bits:) plus the
 *                            optional "+ bias" of QuantizedLinear / MfLinear
 *                            `model/minimax h3/H3Common.swift:358-368`,
 *                            `model/3模块/ltx2.5专属/gemma4文本-(ltx专属).swift:306-312`
 *   mxq_quantized_matmul_ws <- the same call with a caller workspace, into which a
 *                            large-M call tiles the weight first (same result bits)
 *   mxq_qmm, mxq_qmv      <- the two halves of that op (large-M MFMA kernel,
 *                            small-M GEMV kernel), callable directly
 *   mxq_pack, mxq_unpack  <- the packed-code layout itself (no MLX-Swift
 *                            function; the layout of `weight` in the triple
 *                            `model/minimax h3/H3Common.swift:280-281, 389-394`)
 *   mxq_qmm_tiled_act     <- geluApprox(proj_in(x)) of the LTX feed-forward and
 *                            silu(gate) * up of the H3 MLP, fused into the
 *                            matmul's epilogue (mxq_qmm_tiled_lora: plus the
 *                            LoRA term, `model/minimax h3/H3Common.swift:369-375`)
 *                            `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:392-401`,
 *                            `model/minimax h3/H3Transformer.swift:620-629`
 *
 * Conventions (mirroring mlx-c: int status, out-parameters, no exceptions):
 *   - Every function returns MXQ_OK (0) or a negative MXQ_ERR_* code; the
 *     message for the last error on the calling thread is mxq_last_error().
 *   - All tensor pointers are DEVICE pointers, row-major and contiguous,
 *     owned by the caller. Functions enqueue on `stream` (a hipStream_t;
 *     NULL = the default stream) and return without synchronising.
 *   - No function allocates device memory, except mxq_malloc (below) and the
 *     stream-ordered workspace of an MFMA-path mxq_quantized_matmul call (there).
 *   - Packed layout: for output row n, code k occupies bits [k*bits, k*bits+bits)
 *     of the little-endian bitstream formed by wq[n, 0..K*bits/32).
 *     scales, biases: [rows, K/group_size]; w = q*scale + bias.
 *   - bits in {2,3,4,5,6,8}; group_size in {32,64,128}; K % group_size == 0.
 *   - Pointers must be at least 4-byte aligned (MXQ_ERR_ALIGNMENT otherwise).
 */
#ifndef MXQ_H
#define MXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXQ_ABI_VERSION 1

/* status codes */
#define MXQ_OK 0
#define MXQ_ERR_INVALID (-1)     /* shapes, bits, group size or dtype rejected (mlx would throw) */
#define MXQ_ERR_UNSUPPORTED (-2) /* valid mlx arguments this library does not implement */
#define MXQ_ERR_ALIGNMENT (-3)   /* a pointer is not 4-byte aligned */
#define MXQ_ERR_NULL (-4)        /* a required pointer is NULL */
#define MXQ_ERR_HIP (-5)         /* the HIP runtime reported an error */

/* element types */
#define MXQ_FLOAT32 0
#define MXQ_BFLOAT16 1

/* quantizer modes */
#define MXQ_MODE_MINMAX 0   /* scale=(max-min)/(2^bits-1), bias=min */
#define MXQ_MODE_MLX_EDGE 1 /* mlx's sign-aware edge quantizer (as recalled) */

/* Largest M served by the GEMV kernel when mxq_quantized_matmul dispatches: one pass of
 * the weight serves up to 32 tokens (K % 64 == 0; other K: passes of 8 tokens). */
#define MXQ_QMV_MAX_M 32

typedef void* mxq_stream; /* hipStream_t */

/* Quantize w [rows, cols] (w_dtype MXQ_FLOAT32 or MXQ_BFLOAT16) into
 * wq uint32 [rows, cols*bits/32] and scales/biases [rows, cols/group_size]
 * (sb_dtype MXQ_FLOAT32 or MXQ_BFLOAT16). Codes are computed from the fp32
 * scale and bias; the stored scale/bias are then rounded to sb_dtype.
 * Replaces `quantized(w, groupSize:, bits:)` (mlx `quantize`), reached in the
 * reference at `model/minimax h3/tools/quantize_h3_g64.py:132`. */
int mxq_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int group_size,
                 int bits, int mode, uint32_t* wq, void* scales, void* biases,
                 int sb_dtype, mxq_stream stream);

/* out [rows, cols] (out_dtype MXQ_FLOAT32 or MXQ_BFLOAT16) = q*scale + bias,
 * evaluated as one fp32 fused multiply-add, then rounded to out_dtype (RNE).
 * Replaces `dequantized(...)` / MfLinear.dequantizedWeight
 * (`model/minimax h3/H3Common.swift:382-401`, which is 4-bit only; this
 * handles every supported width). */
int mxq_dequantize(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                   int64_t rows, int64_t cols, int group_size, int bits, void* out,
                   int out_dtype, mxq_stream stream);

/* Pack codes uint8 [rows, cols] (each < 2^bits) into wq uint32 [rows, cols*bits/32].
 * Codes >= 2^bits are masked to their low `bits` bits. */
int mxq_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
             mxq_stream stream);

/* Unpack wq uint32 [rows, cols*bits/32] into codes uint8 [rows, cols]. */
int mxq_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits, uint8_t* codes,
               mxq_stream stream);

/* y bf16 [M, N] = x bf16 [M, K] * dequant(wq, scales, biases)^T (+ bias bf16 [N]).
 * scales/biases bf16 [N, K/group_size]; fp32 accumulation; bias may be NULL.
 * transpose must be 1 (the only form the reference uses,
 * `model/minimax h3/H3Common.swift:358-359`); transpose == 0 returns
 * MXQ_ERR_UNSUPPORTED. M <= 8 runs the GEMV kernel; 9 <= M <= MXQ_QMV_MAX_M (K % 64 ==
 * 0) the GEMV or an MFMA kernel, whichever an estimate from the weight's size and K
 * finds faster; larger M an MFMA kernel. M == 0 or N == 0 is a no-op.
 * When an MFMA kernel runs and K % 64 == 0 (and the tiled copy is below 2 GiB) the call takes
 * mxq_tiled_bytes(N, K, group_size, bits) bytes of stream-ordered workspace from a memory
 * pool the library owns (one per GPU, created on first use, kept until the process ends,
 * caching up to 256 MiB of freed workspace), tiles the weight into it, runs the tiled MFMA
 * kernel and frees the workspace on `stream`: the same result bits as the in-place MFMA
 * kernel. On a stream under graph capture, or where the pool cannot supply the bytes, it
 * runs the in-place kernel and allocates nothing. */
int mxq_quantized_matmul(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                         const void* scales, const void* biases, int64_t N, int transpose,
                         int group_size, int bits, const void* bias, void* y,
                         mxq_stream stream);

/* mxq_quantized_matmul with a caller-provided workspace, for callers that keep the
 * weight in the MLX layout (the same `quantizedMM` call,
 * `model/minimax h3/H3Common.swift:358-359`). When
 * mxq_quantized_matmul_workspace_size(M, N, K, group_size, bits) is positive and the
 * workspace holds that many bytes (16-byte aligned), the weight is first tiled into it
 * (mxq_tile) and the tiled MFMA kernel runs: bit-identical results, about 1.6x faster
 * at M = 14400, K = 4096, N = 16384. Otherwise, including a NULL or too small
 * workspace, this is mxq_quantized_matmul's in-place form (the GEMV or the in-place
 * MFMA kernel). Allocates nothing; the workspace is
 * overwritten, and calls sharing one workspace must be ordered on one stream. A
 * workspace that overlaps x, the weight triple, bias or y is MXQ_ERR_INVALID.
 * The size is positive only for M >= 1024 and K % 64 == 0; a negative return is an
 * MXQ_ERR_* code for invalid bits / group_size / K / M. */
int64_t mxq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size,
                                            int bits);
int mxq_quantized_matmul_ws(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                            const void* scales, const void* biases, int64_t N, int transpose,
                            int group_size, int bits, const void* bias, void* y, void* workspace,
                            size_t ws_bytes, mxq_stream stream);

/* mxq_quantized_matmul_ws for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The workspace is a static device array of MXQ_NOALLOC_SCRATCH_BYTES,
 * one per GPU, held by the library until the process ends; nothing is allocated
 * and nothing is freed. When the tiled path applies (workspace_size > 0) and the
 * tiled weight fits, the weight is tiled into that array and the tiled kernel runs
 * (the same result bits as mxq_quantized_matmul); when it does not apply, this is
 * mxq_quantized_matmul's in-place form (nothing allocated); a tiled weight above the
 * array's size is MXQ_ERR_INVALID.
 * Every call on one GPU shares that GPU's array: calls that may overlap on one GPU
 * (different streams, not ordered) race and must be serialised by the caller. */
#define MXQ_NOALLOC_SCRATCH_BYTES (64ll << 20)
int mxq_quantized_matmul_noalloc(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                                 const void* scales, const void* biases, int64_t N,
                                 int transpose, int group_size, int bits, const void* bias,
                                 void* y, mxq_stream stream);

/* Large-M path only (bf16 MFMA, weights unpacked in registers). Any M >= 0. */
int mxq_qmm(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* scales,
            const void* biases, int64_t N, int group_size, int bits, const void* bias,
            void* y, mxq_stream stream);

/* Small-M path only (the GEMV kernels). 0 <= M <= MXQ_QMV_MAX_M. */
int mxq_qmv(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* scales,
            const void* biases, int64_t N, int group_size, int bits, const void* bias,
            void* y, mxq_stream stream);

/* ---- tiled weight layout ----------------------------------------------------
 * A load-time reordering of the same packed bits (no requantization) in which
 * every weight load of both kernels is a coalesced 16-byte-per-lane access:
 * records of (64 output rows x 64 codes) in step-major order (the records of one
 * 64-code K step, all row blocks, are adjacent), each record holding the codes in
 * lane order followed by one (scale, bias) bf16 pair per lane unit. Rows past N
 * are zero. Requires K % 64 == 0 and bf16 scales/biases; the tiled copy stays
 * below 2 GiB (mxq_tiled_bytes is MXQ_ERR_INVALID above).
 * The MLX-layout entry points above remain the drop-in operators; the tiled
 * ones are what QuantizedLinear uses once its weights are resident (the
 * reference keeps weights resident the same way: H3Weights / MfLinear.load,
 * `model/minimax h3/H3Common.swift:312-338`). No reference counterpart exists
 * for the layout itself. */

/* Bytes needed for the tiled copy of an N x K weight; negative on invalid
 * arguments or a copy of 2 GiB or more (then mxq_last_error() says why). */
int64_t mxq_tiled_bytes(int64_t N, int64_t K, int group_size, int bits);

/* MLX layout (wq, scales, biases; bf16 scales/biases) -> tiled layout. */
int mxq_tile(const uint32_t* wq, const void* scales, const void* biases, int64_t N, int64_t K,
             int group_size, int bits, void* tiled, mxq_stream stream);

/* mxq_quantized_matmul on tiled weights: the GEMV or the MFMA kernel by the same rule as
 * mxq_quantized_matmul. Same arithmetic and results as the MLX-layout paths. */
int mxq_quantized_matmul_tiled(const void* x, int64_t M, int64_t K, const void* tiled,
                               int64_t N, int group_size, int bits, const void* bias, void* y,
                               mxq_stream stream);

/* The two halves of mxq_quantized_matmul_tiled, callable directly. */
int mxq_qmm_tiled(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                  int group_size, int bits, const void* bias, void* y, mxq_stream stream);
int mxq_qmv_tiled(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                  int group_size, int bits, const void* bias, void* y, mxq_stream stream);

/* ---- activations fused into the tiled MFMA kernel's epilogue ---------------
 * The activation is applied to x*W^T + bias in fp32, before the single bf16
 * rounding, so the pre-activation [M, N] never goes to memory. */
#define MXQ_ACT_NONE 0
#define MXQ_ACT_GELU_TANH 1 /* 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))) */
#define MXQ_ACT_SWIGLU 2    /* silu(gate) * up, weights tiled by mxq_tile_swiglu */

/* Tiled layout of an [N, K] weight whose rows are [gate; up] (N even, N/2 rows
 * each): record row block rb holds gate rows 32rb .. 32rb+31 in its first half
 * and the matching up rows N/2 + 32rb .. N/2 + 32rb+31 in its second, so that
 * one lane holds both operands of silu(gate) * up. Same size as
 * mxq_tiled_bytes(N, ...). Serves the fused fc1 of the H3 MLP, whose output the
 * reference splits in halves and combines as silu(gate) * up
 * (`model/minimax h3/H3Transformer.swift:620-629`). */
int mxq_tile_swiglu(const uint32_t* wq, const void* scales, const void* biases, int64_t N,
                    int64_t K, int group_size, int bits, void* tiled, mxq_stream stream);

/* Tiled layout -> MLX layout (wq [N, K*bits/32], bf16 scales and biases [N, K/gs]),
 * the inverse of mxq_tile / mxq_tile_swiglu: the same bits come back. For holders
 * that keep only the tiled copy resident and rebuild the triple when it is asked
 * for: the reference's QuantizedLinear parameters weight / scales / biases
 * (`model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188`) and MfLinear's
 * dequantizedWeight() (`model/minimax h3/H3Common.swift:382-401`). */
int mxq_untile(const void* tiled, int64_t N, int64_t K, int group_size, int bits, uint32_t* wq,
               void* scales, void* biases, mxq_stream stream);
int mxq_untile_swiglu(const void* tiled, int64_t N, int64_t K, int group_size, int bits,
                      uint32_t* wq, void* scales, void* biases, mxq_stream stream);

/* y = act(x * W^T + bias) on the MFMA kernel, any M >= 0:
 *   MXQ_ACT_NONE       as mxq_qmm_tiled;
 *   MXQ_ACT_GELU_TANH  weights from mxq_tile; y [M, N]. Replaces
 *                      geluApprox(proj_in(x)) between the LTX feed-forward
 *                      projections (`model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:392-401`);
 *   MXQ_ACT_SWIGLU     weights from mxq_tile_swiglu, N even, bias [N] (gate
 *                      half, then up half); y [M, N/2] = silu(gate) * up
 *                      (`model/minimax h3/H3Transformer.swift:620-629`). */
int mxq_qmm_tiled_act(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                      int group_size, int bits, const void* bias, int act, void* y,
                      mxq_stream stream);

/* mxq_qmm_tiled_act plus a rank-R update added to the fp32 accumulators before the
 * bias, the activation and the rounding: y = act(x*W^T + bias + xa*bt^T). This is
 * the LoRA term of the reference's MfLinear.forward, out + sum_i scale_i (x A_i) B_i
 * (`model/minimax h3/H3Common.swift:369-375, 421-434`): xa bf16 [M, R] = x [A_1 | A_2
 * | ...] (the caller's small GEMM), bt bf16 [N, R] = [scale_1 B_1; scale_2 B_2; ...]^T,
 * rows in the weight's row order ([gate; up] for MXQ_ACT_SWIGLU). R a positive
 * multiple of 16 (zero-pad the adapters), at most 4096. xa == bt == NULL, R == 0:
 * no update. */
int mxq_qmm_tiled_lora(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                       int group_size, int bits, const void* bias, int act, const void* xa,
                       const void* bt, int64_t R, void* y, mxq_stream stream);

/* ---- row-wise ops of the DiT block around the linears -----------------------
 * The H3 block's fused kernels (`model/2网络算子/网络算子-融合-RMSNormRoPE-通用.swift:41-343`,
 * called at `model/minimax h3/H3Transformer.swift:455-480, 1117-1155`), with their
 * arithmetic: fp32 mean of squares, rsqrt, the normalised value rounded to bf16,
 * then the modulation or rotation in fp32 and one more bf16 rounding. x, other,
 * weight, shift, scale, gate and out are bf16; row_map [S] picks the modulation
 * row of each token row (NULL: row 0; entries past mod_rows - 1 are clamped).
 * HBM-bound; one wave per row. */

/* out [S, hidden] = (rmsnorm(x) * weight) * (scale[m] + 1) + shift[m]:
 * rmsNormLast + modScaleShift (fusedNormModscale / fusedNormModscaleRow);
 * shift, scale [mod_rows, hidden]. */
int mxq_norm_modscale(const void* x, int64_t S, int64_t hidden, const void* weight,
                      const void* shift, const void* scale, int64_t mod_rows,
                      const uint32_t* row_map, float eps, void* out, mxq_stream stream);

/* out [S, hidden] = x + other * gate[m] (fusedModGate); gate [mod_rows, hidden]. */
int mxq_mod_gate(const void* x, const void* other, int64_t S, int64_t hidden, const void* gate,
                 int64_t mod_rows, const uint32_t* row_map, void* out, mxq_stream stream);

/* out [S, heads, head_dim] = split-half rotary of rmsnorm(x) * weight over the last axis
 * (fusedRmsnormRope = rmsNormLast + applyRopePub, `H3Common.swift:502-508, 555-569`): for
 * j < rot/2, (n_j, n_{j+rot/2}) rotate by the angle of (token, j); dims >= rot pass
 * through. weight [head_dim]; cos, sin [S, rot/2] in table_dtype (MXQ_FLOAT32 or
 * MXQ_BFLOAT16). head_dim <= 512, rot even, rot <= head_dim. */
int mxq_rmsnorm_rope(const void* x, int64_t S, int64_t heads, int64_t head_dim,
                     const void* weight, const void* cos, const void* sin, int table_dtype,
                     int rot, float eps, void* out, mxq_stream stream);

/* ---- safetensors files (read-only) -----------------------------------------
 * The on-disk form of the quantized triples: `prefix.weight` U32 packed codes
 * plus `prefix.scales` / `prefix.biases` (or `prefix.weight.scales` /
 * `.weight.biases`), as the reference's H3Weights reads them: header parsed
 * once, tensors read on demand (`model/minimax h3/H3Common.swift:181-260`),
 * file mapped read-only (`model/3模块/Safetensors-mmap映射-通用.swift:40-135`).
 * A handle is not thread-safe. */
#define MXQ_ST_MAX_DIMS 8
typedef struct mxq_safetensors mxq_safetensors;

/* Maps `path` and parses its header; MXQ_ERR_INVALID for a missing file or a
 * malformed header (sizes and ranges are checked against the file). */
int mxq_st_open(const char* path, mxq_safetensors** out);
/* Waits for the handle's pending copies, then unmaps and frees it. */
void mxq_st_close(mxq_safetensors* st);
/* Number of tensors and the i-th key (header order). */
int64_t mxq_st_count(const mxq_safetensors* st);
const char* mxq_st_key(const mxq_safetensors* st, int64_t i);
/* dtype name ("U32", "BF16", ...), rank, shape and byte size of `key`. */
int mxq_st_info(const mxq_safetensors* st, const char* key, char dtype[16], int* ndim,
                int64_t shape[MXQ_ST_MAX_DIMS], int64_t* nbytes);
/* Copies the tensor's bytes to host memory. */
int mxq_st_read_host(const mxq_safetensors* st, const char* key, void* dst);
/* Enqueues the tensor's bytes to device memory `dst` on `stream`: the mapped
 * bytes are staged through two pinned host buffers (held by the handle, freed
 * at close), so reading chunk i+1 from the file overlaps the copy of chunk i.
 * Returns once every chunk is staged; the file may then be closed. */
int mxq_st_read(mxq_safetensors* st, const char* key, void* dst, mxq_stream stream);

/* Message of the last failed call on this thread ("" if none). */
const char* mxq_last_error(void);

/* Short name of a status code. */
const char* mxq_status_string(int status);

/* Blocks until all work on `stream` has finished; reports asynchronous kernel
 * errors as MXQ_ERR_HIP. */
int mxq_stream_synchronize(mxq_stream stream);

/* ---- device memory and streams, for hosts that do not link HIP themselves ----
 * (the Swift bridge, C programs). The reference's rule for buffers holds here:
 * free device memory only after the work that uses it has finished, i.e. after
 * synchronizing the stream it was used on (`model/minimax h3/H3Pipeline.swift:
 * 212-228`, Stream.gpu.synchronize() before buffers are released). */
int mxq_stream_create(mxq_stream* stream); /* a new stream of default priority */
int mxq_stream_destroy(mxq_stream stream); /* NULL: no-op */
int mxq_malloc(void** ptr, size_t bytes);  /* device memory; bytes == 0 gives NULL */
int mxq_free(void* ptr);                   /* NULL: no-op */
/* Copies between host and device memory on `stream`; both return once the copy
 * (and all earlier work on the stream) has finished, so `src` may then be reused. */
int mxq_copy_to_device(void* dst, const void* src, size_t bytes, mxq_stream stream);
int mxq_copy_to_host(void* dst, const void* src, size_t bytes, mxq_stream stream);

/* MXQ_ABI_VERSION of the loaded library. */
int mxq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MXQ_H */
